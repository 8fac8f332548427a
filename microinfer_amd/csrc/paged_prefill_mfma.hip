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
//    online softmax needs a cross-lane exchange only when the running
//    maximum moves and once for the row sum at the end.
//  * O^T += V^T . P^T on the same instruction: P^T comes straight from the
//    softmax registers. The MFMA reduction index is mapped to keys the way
//    the S^T result lays them out; the V^T fragments are read from the
//    row-major V tile with transposing LDS reads (ds_read_b64_tr_b16), so
//    neither P nor V is shuffled.
//  * K/V tiles move from global memory straight into LDS (buffer or global
//    loads with the LDS flag: no staging registers, no LDS store
//    instructions) through three LDS buffers, two tiles ahead of the one being
//    computed; the tile loop is unrolled by three so every LDS address is a
//    register plus an immediate. One barrier per tile; at most 168 VGPRs, so
//    three workgroups (12 waves) share a CU.
//  * Per tile and wave the scalar work is one block-id load, a multiply-add
//    for the block's offset (the scalar offset of buffer loads from the
//    head's K and V bases) and three M0 writes.
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

// Two packed 1.0 values of the element type (for row sums with dot2).
template <typename E>
constexpr uint32_t kOnes2 = std::is_same<E, BF16>::value ? 0x3F803F80u : 0x3C003C00u;

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
constexpr int kWaves = 4;             // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kTileElems = kKeys * kD;  // one K or V tile in LDS (8 KiB of bf16)
// Rows of a tile each wave moves with direct global->LDS loads (4 rows of
// 256 bytes per instruction).
constexpr int kRowsPerWave = kKeys / kWaves;
static_assert(kWaves == 4 && kRowsPerWave % 4 == 0, "tile load mapping");

// LDS tile layouts (LDS serves 256 bytes per clock, so an access is
// conflict-free when each group of lanes served together covers 256
// distinct bytes):
//  * K: [key half][16-byte chunk][16 keys]. A K fragment read (16 lanes x
//    16 bytes: keys k..k+15 of one half, one chunk) covers 256 contiguous
//    bytes, and the reads of successive k-steps are 512 bytes apart, so
//    each is one register plus an immediate offset.
//  * V: key rows of 256 bytes, row-major, with the 16-byte chunk c of key k
//    stored at position c ^ swz_v(k). The transposed reads (32 lanes x 8
//    bytes: 4 consecutive keys x 4 aligned chunks) need the 4 keys' chunk
//    groups disjoint: swz_v(k) = 4 * (k & 3).
__device__ __forceinline__ int swz_v(int key) { return 4 * (key & 3); }

// A (row block, KV head) split along its keys has at most kMaxParts
// partitions; the last one to finish merges them kMergeBatch at a time.
constexpr int kMaxParts = 8;
constexpr int kMergeBatch = 4;

// Largest exponent a probability may reach before the running maximum is
// moved (p <= 2^15 fits f16 as well as bf16).
constexpr float kRescaleSlack = 15.f;

typedef short short4_t __attribute__((ext_vector_type(4)));
using LdsShort4 = __attribute__((address_space(3))) short4_t;
using LdsVoid = __attribute__((address_space(3))) void;

// Four 16-bit elements, transposed across each group of 16 lanes
// (ds_read_b64_tr_b16): lane l of a group receives element l % 4 of the
// 8-byte rows read by lanes l / 4, l / 4 + 4, l / 4 + 8 and l / 4 + 12.
__device__ __forceinline__ short4_t read_tr(const uint16_t* lds_elem) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsShort4*)(lds_elem));
}

// Buffer resource (V#) over `base`: raw (stride 0) with the largest record
// count, so addresses are base + soffset + lane offset + instruction offset
// with no range clamp (the kernel keeps every offset inside the cache).
typedef int32_t BufRsrc __attribute__((ext_vector_type(4)));
__device__ __forceinline__ BufRsrc make_buf_rsrc(const void* base) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  BufRsrc r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(p));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int32_t>((p >> 32) & 0xFFFFu));
  r.z = -1;           // num_records
  r.w = 0x00020000;   // 32-bit data format, no swizzle
  return r;
}

// One direct buffer->LDS load of 16 bytes per lane: lane i writes LDS bytes
// lds_dst + 16 i from rsrc + soff + voff (one wait state after the M0
// write). Untracked by the compiler, like lds_load16.
__device__ __forceinline__ void lds_load16_buf(BufRsrc rsrc, uint32_t soff, uint32_t voff,
                                               const void* lds_dst) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) void*)(lds_dst)));
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
               : "memory", "m0");
}

// Two direct buffer->LDS loads of 16 bytes per lane sharing one M0 (one
// wait state after the M0 write): lane i of the first writes LDS bytes
// lds_dst + 16 i from rsrc + soff + voff0; the second's instruction offset
// 1024 is added to both addresses, so it writes lds_dst + 1024 + 16 i from
// rsrc + soff + voff1m + 1024. Untracked by the compiler, like lds_load16.
__device__ __forceinline__ void lds_load16x2_buf(BufRsrc rsrc, uint32_t soff, uint32_t voff0,
                                                 uint32_t voff1m, const void* lds_dst) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) void*)(lds_dst)));
  asm volatile(
      "s_mov_b32 m0, %4\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %0, %2, %3 offen lds\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen offset:1024 lds"
      :
      : "v"(voff0), "v"(voff1m), "s"(rsrc), "s"(soff), "s"(lds)
      : "memory", "m0");
}

// ---------------------------------------------------------------------------
// Single-row requests (the decode rows of a mixed batch). A 32-row query
// block gives the one row 1/32 of its MFMA and softmax work and takes as
// long as a 32-row block of a long chunk, so these requests take a path of
// their own in the same launch: one workgroup per (request, KV head) streams
// the request's context in 16-position tiles, wave w taking tiles w, w + 4,
// ... through its own LDS slot (direct loads, one tile in flight per wave),
// with the G query heads as the columns of 16x16 MFMAs: S^T[pos][head] =
// K . Q^T on 16x16x32 (A = a K row per lane, B = the query rows, heads >= G
// zero), whose result puts 4 positions of one head in each lane -- the
// B-operand layout of O^T[dim][head] += V^T . P^T on 16x16x16, with V^T
// read from the row-major tile by transposing LDS reads. The four waves'
// states are combined through LDS at the end.
// ---------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

template <typename E>
struct RowMfma;
template <>
struct RowMfma<BF16> {
  static __device__ __forceinline__ f32x4_t qk(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(short4_t a, short4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <>
struct RowMfma<F16> {
  static __device__ __forceinline__ f32x4_t qk(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(short4_t a, short4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
};

constexpr int kRowTile = 16;                     // positions per single-row tile
constexpr int kRowBytes = kD * 2;                // one cache row (256 bytes)
constexpr int kRowHalf = kRowTile * kRowBytes;   // K (or V) of one tile: 4 KiB
constexpr int kRowSlot = 2 * kRowHalf;           // K then V: 8 KiB per wave
static_assert(kWaves * kRowSlot <= 2 * 3 * kTileElems * 2, "slots fit the tile ring");

// Slot rows are 256 bytes with the 16-byte chunk c of row r at position
// c ^ swz(r): K fragment reads (16 lanes: rows 0-15, one chunk each) are
// conflict-free with r & 15, the transposed V reads (32 lanes: rows r..r+7,
// two adjacent chunks each) with 2 (r & 7).
__device__ __forceinline__ int row_swz_k(int r) { return r & 15; }
__device__ __forceinline__ int row_swz_v(int r) { return 2 * (r & 7); }

__device__ __forceinline__ float lane_xor16(float v, int lane) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
}

// Attention of request `req`'s single query row (row `q_row`) over its `ctx`
// paged keys for KV head `head`, all G query heads, written to the output.
// `slots`: kWaves x kRowSlot bytes of LDS; s_m / s_l: [kWaves][16] floats.
template <typename E, int G>
__device__ __forceinline__ void single_row_attention(const AttnArgs& a, int req, int head,
                                                     int q_row, int ctx, char* slots,
                                                     float (*s_m)[16], float (*s_l)[16]) {
  using M = RowMfma<E>;
  using vec8 = typename Mfma<E>::vec8;
  using R = uint16_t;
  using ConstI32 = __attribute__((address_space(4))) const int32_t;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int col = lane % 16;   // MFMA column: query head within the group
  const int quad = lane / 16;  // positions 4 quad .. 4 quad + 3 of a tile
  const int ntiles = (ctx + kRowTile - 1) / kRowTile;
  const ConstI32* ctab = (const ConstI32*)(a.tables + req * a.t_stride);
  const R* kc = static_cast<const R*>(a.kc);
  const R* vc = static_cast<const R*>(a.vc);
  const int64_t head_off = static_cast<int64_t>(head) * a.c_hs;
  const int c_ts = static_cast<int>(a.c_ts);
  // Direct load u of a half-tile puts lane i's 16 bytes at slot row
  // 4u + i / 16, chunk position i % 16 (logical chunk (i % 16) ^ swz(row)).
  uint32_t off_k[4], off_v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 4 * u + lane / 16;
    off_k[u] = static_cast<uint32_t>((row * c_ts + ((lane % 16) ^ row_swz_k(row)) * 8) * 2);
    off_v[u] = static_cast<uint32_t>((row * c_ts + ((lane % 16) ^ row_swz_v(row)) * 8) * 2);
  }
  char* slot = slots + wave * kRowSlot;
  // Issue tile k's loads; returns whether its block id is valid (an invalid
  // block reads block 0 and is masked).
  auto issue = [&](int k) -> bool {
    const int p0 = k * kRowTile;
    const int blk = ctab[p0 >> a.log2_block];
    const bool ok = static_cast<uint32_t>(blk) < static_cast<uint32_t>(a.num_blocks);
    const int64_t base = (ok ? static_cast<int64_t>(blk) * a.c_bs +
                                   static_cast<int64_t>(p0 & (a.block_size - 1)) * a.c_ts
                             : 0) + head_off;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      lds_load16_sbase(kc + base, off_k[u], slot + u * kWave * 16);
      lds_load16_sbase(vc + base, off_v[u], slot + kRowHalf + u * kWave * 16);
    }
    return ok;
  };

  int k = wave;
  bool ok = false;
  if (k < ntiles) ok = issue(k);
  // Query fragments (B operand): k-step ks holds dims 32 ks + 8 quad .. +7
  // of head `col` (zero for col >= G).
  vec8 qf[kD / 32];
  {
    const R* qrow = static_cast<const R*>(a.q) + q_row * a.q_ts + (head * G + col) * a.q_hs;
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      Pack<R, 8> pq = zero_pack<R, 8>();
      if (col < G) pq = load_pack<R, 8>(qrow + ks * 32 + quad * 8);
      qf[ks] = __builtin_bit_cast(vec8, pq);
    }
  }
  f32x4_t o[kD / 16];
#pragma unroll
  for (int db = 0; db < kD / 16; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale_log2;
  for (; k < ntiles; k += kWaves) {
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this wave's tile and Q
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int p0 = k * kRowTile;
    // Rows past the context or of an invalid block hold whatever the cache
    // holds there: weight 0, but 0 * NaN is NaN, so their V rows are zeroed.
    if (!ok || p0 + kRowTile > ctx) {
      const int r = lane / 4;
      if (!ok || p0 + r >= ctx) {
        char* row = slot + kRowHalf + r * kRowBytes + (lane % 4) * 64;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<Pack<uint32_t, 4>*>(row + c * 16) = zero_pack<uint32_t, 4>();
      }
    }
    vec8 kf[kD / 32];
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      const int chunk = (4 * ks + quad) ^ row_swz_k(col);
      kf[ks] = __builtin_bit_cast(
          vec8, *reinterpret_cast<const Pack<R, 8>*>(slot + col * kRowBytes + chunk * 16));
    }
    short4_t vf[kD / 16];
    {
      const int vrow = 4 * quad + col / 4;
      const char* vbase = slot + kRowHalf + vrow * kRowBytes + 8 * (col & 1);
#pragma unroll
      for (int db = 0; db < kD / 16; ++db) {
        const int chunk = (2 * db + ((col % 4) >> 1)) ^ row_swz_v(vrow);
        vf[db] = read_tr(reinterpret_cast<const uint16_t*>(vbase + chunk * 16));
      }
    }
    f32x4_t sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) sv = M::qk(kf[ks], qf[ks], sv);
    // sv[i]: score of position p0 + 4 quad + i for head `col`.
    const int p = p0 + 4 * quad;
    float sc[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (ok && p + i < ctx) ? sv[i] * scale_log2 : -INFINITY;
      tmax = fmaxf(tmax, sc[i]);
    }
    tmax = fmaxf(tmax, lane_xor16(tmax, lane));
    tmax = fmaxf(tmax, partner32(tmax, lane));
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
      pk.v[i] = to_raw<E>(fast_exp2(sc[i] + neg_m));
      l += E::load(pk.v[i]);  // the weight the MFMA applies
    }
    const short4_t pf = __builtin_bit_cast(short4_t, pk);
#pragma unroll
    for (int db = 0; db < kD / 16; ++db) o[db] = M::pv(vf[db], pf, o[db]);
    if (k + kWaves < ntiles) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot's reads returned
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      ok = issue(k + kWaves);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // every load landed before the slot is reused
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // Per-head row sum over the four position groups.
  l += lane_xor16(l, lane);
  l += partner32(l, lane);
  // Wave states to LDS: acc[h][d] floats in the wave's own (drained) slot.
  float* my_acc = reinterpret_cast<float*>(slot);
  if (col < G) {
#pragma unroll
    for (int db = 0; db < kD / 16; ++db)
      *reinterpret_cast<f32x4_t*>(my_acc + col * kD + db * 16 + 4 * quad) = o[db];
  }
  if (lane < 16) {
    s_m[wave][lane] = m;
    s_l[wave][lane] = l;
  }
  __syncthreads();
  // Combine the waves: thread e handles (h, d) = (e / 128, e % 128).
  R* out = static_cast<R*>(a.out) + q_row * a.o_ts + (head * G) * a.o_hs;
  constexpr int kElems = G * kD;
#pragma unroll
  for (int e = tid; e < kElems; e += kThreads) {
    const int h = e / kD, d = e % kD;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][h]);
    float ls = 0.f, os = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_m[w][h];
      const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - mx);
      ls = fmaf(f, s_l[w][h], ls);
      os = fmaf(f, reinterpret_cast<const float*>(slots + w * kRowSlot)[h * kD + d], os);
    }
    const float inv = ls > 0.f ? 1.f / ls : 0.f;
    out[h * a.o_hs + d] = E::store(os * inv);
  }
}

// A32: every element offset into the caches fits in int32 (checked on the
// host), so tile offsets are 32-bit (buffer loads for paged caches); the
// 64-bit forms cost about 4 % of the kernel in scalar issue slots.
// PAGED: block tables given (else contiguous K/V rows, cu_k offsets).
template <typename E, int G, bool A32, bool PAGED>
__global__ __launch_bounds__(kThreads, 3) void paged_prefill_mfma_kernel(const AttnArgs a) {
  using M = Mfma<E>;
  using vec8 = typename M::vec8;
  using R = uint16_t;
  constexpr int BM = kRows * kWaves / G;  // query rows per workgroup
  using ConstI32 = __attribute__((address_space(4))) const int32_t;
  // Three K/V tile buffers (48 KiB per workgroup), K in the first three
  // tiles, V in the last three; single-row requests use them as four 8 KiB
  // slots.
  __shared__ __attribute__((aligned(16))) R s_kv[6][kTileElems];
  __shared__ float s_row_m[kWaves][16];
  __shared__ float s_row_l[kWaves][16];
  __shared__ int s_arrived;
  R(*s_k)[kTileElems] = s_kv;
  R(*s_v)[kTileElems] = s_kv + 3;

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
  // With a plan, the workgroup's item says it all: request, row block, key
  // tiles and, for a (row block, KV head) split along its keys, the
  // partition and where its partial goes.
  const ConstI32* cu_q = (const ConstI32*)(a.cu_q);
  const ConstI32* cu_k = (const ConstI32*)(a.cu_k);
  int req = -1, qb0 = 0, rblock = 0;
  int t_begin = 0, t_end = INT_MAX, part = 0, nparts = 1, slot = 0, counter = 0;
  if (a.prefill_plan != nullptr) {
    if (qblock >= *(const ConstI32*)(a.prefill_count)) return;  // surplus (uniform)
    const ConstI32* it = (const ConstI32*)(a.prefill_plan + qblock);
    req = it[0];
    rblock = it[1];
    t_begin = it[2];
    t_end = it[3];
    part = it[4];
    nparts = it[5];
    slot = it[6];
    counter = it[7];
  } else {
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
    // Within a request the last query block (the most keys) runs first.
    rblock = (cu_q[req + 1] - cu_q[req] + BM - 1) / BM - 1 - (qblock - qb0);
  }
  const int q_begin = cu_q[req];
  const int q_len = cu_q[req + 1] - q_begin;
  constexpr bool paged = PAGED;  // block tables given (else contiguous K/V)
  int ctx = cu_k[req + 1] - cu_k[req];
  if (paged) ctx = min(ctx, a.t_width * a.block_size);
  const int64_t krow0 = paged ? 0 : cu_k[req];
  if constexpr (PAGED) {
    if (q_len == 1 && nparts == 1) {  // uniform across the workgroup
      single_row_attention<E, G>(a, req, head, q_begin, ctx, reinterpret_cast<char*>(s_kv),
                                 s_row_m, s_row_l);
      return;
    }
  }
  const int wg_row0 = rblock * BM;
  const int wg_last = min(q_len, wg_row0 + BM) - 1;
  // Keys the workgroup needs: up to the causal limit of its last row.
  int kv_end = max(0, min(ctx, ctx - q_len + wg_last + 1));
  if (!paged) kv_end = static_cast<int>(min<int64_t>(kv_end, max<int64_t>(a.num_blocks - krow0, 0)));
  // This workgroup's tiles: [t_begin, ntiles) of the row block's.
  const int ntiles = min((kv_end + kKeys - 1) / kKeys, t_end);
  t_begin = min(t_begin, ntiles);
  const int nfull = kv_end / kKeys;  // tiles wholly below kv_end

  const int my_row = wg_row0 + rsub * kRows + col;  // row within the request
  const bool row_ok = my_row < q_len && rsub * kRows < BM;
  const int qpos = ctx - q_len + my_row;  // this row sees keys 0 .. qpos
  // Causal limit of the wave's first row (the smallest of the wave's rows):
  // tiles below nint need no causal or range mask for any row of the wave.
  const int qpos_first = ctx - q_len + wg_row0 + rsub * kRows;
  const int nint = min(nfull, max(qpos_first + 1, 0) / kKeys);

  // Q^T fragments (B operand): k-step ks covers head dims ks*16 .. ks*16+15;
  // this lane supplies dims ks*16 + half*8 .. +7 of its row.
  const R* qrow = static_cast<const R*>(a.q) + (q_begin + my_row) * a.q_ts +
                  (head * G + g) * a.q_hs;
  // Loaded after the first tiles' loads are issued (their latencies overlap);
  // an explicit full wait then leaves the compiler no Q load to wait for
  // inside the loop, where it would also wait for the prefetched tiles.
  vec8 qf[kD / 16];

  // Tile loads go straight from global memory to LDS (direct loads: lane i
  // of an instruction writes bytes 16i .. 16i+15 after the instruction's LDS
  // base, 1 KiB per instruction). Waves 0-1 move the tile's first 16-key
  // half, waves 2-3 the second; each half lies in one cache block (block
  // size >= 16), so a wave's loads share one scalar base and each lane adds
  // a constant offset. Per wave and tile, two K and two V instructions:
  //  * K instruction j: chunks 8 (w % 2) + 4j .. +3 of the half's 16 keys
  //    (lane i: key i % 16, chunk 8 (w % 2) + 4j + i / 16);
  //  * V instruction j: key rows 8w + 4j .. +3 (lane i: row 8w + 4j + i / 16,
  //    LDS chunk position i % 16, i.e. logical chunk (i % 16) ^ swz_v(row)).
  const R* kc = static_cast<const R*>(a.kc);
  const R* vc = static_cast<const R*>(a.vc);
  const int32_t* trow = paged ? a.tables + req * a.t_stride : nullptr;
  const int64_t head_off = static_cast<int64_t>(head) * a.c_hs;
  const int c_ts = static_cast<int>(a.c_ts);
  const int c_bs32 = static_cast<int>(a.c_bs);  // used when A32
  const bool wave_half = wave >= 2;  // which 16-key half of a tile this wave moves
  const int wrow = wave_half ? 16 : 0;
  const int kkey = lane % 16;  // key within the half (K loads)
  int k_ch[2], v_key[2], v_ch[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    k_ch[j] = 8 * (wave % 2) + 4 * j + lane / 16;
    v_key[j] = wave * kRowsPerWave + 4 * j + lane / 16;
    v_ch[j] = (lane % 16) ^ swz_v(v_key[j]);
  }
  // LDS element offsets of the wave's instructions within a tile buffer.
  const int k_lds = (wave_half ? 16 * kD : 0) + (8 * (wave % 2)) * 16 * 8;
  const int v_lds = wave * kRowsPerWave * kD;
  // Byte offsets from the wave's half-tile base (row within the half, then
  // chunk), constant over the whole loop, so a tile's loads need no per-lane
  // address arithmetic.
  uint32_t off_k[2], off_v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    off_k[j] = static_cast<uint32_t>((kkey * c_ts + k_ch[j] * 8) * 2);
    off_v[j] = static_cast<uint32_t>(((v_key[j] % 16) * c_ts + v_ch[j] * 8) * 2);
  }
  // A32 paged loads are buffer loads: the head's K and V bases sit in two
  // buffer resources and a tile's block offset is the scalar soffset. The
  // two V loads share one M0 (the second adds 1024 to both its LDS and
  // memory addresses, so its lane offset is taken 1024 lower: rows 4-7 of a
  // wave's eight lie at least 4 * c_ts * 2 >= 1024 bytes into the block,
  // c_ts >= 128 being checked on the host).
  BufRsrc rsrc_k{}, rsrc_v{};
  if constexpr (A32) {
    if constexpr (paged) {
      rsrc_k = make_buf_rsrc(kc + head_off);
      rsrc_v = make_buf_rsrc(vc + head_off);
    }
  }
  const uint32_t bs_bytes = static_cast<uint32_t>(c_bs32) * 2u;
  const uint32_t ts_bytes = static_cast<uint32_t>(c_ts) * 2u;
  const bool pair_ids = a.block_size == 16;  // a tile's halves lie in two blocks
  // Issue the loads of `tile` into (kbuf, vbuf); returns the tile's mask
  // (bit h: its 16-key half h has a valid block id).
  auto issue_tile = [&](int tile, R* kbuf, R* vbuf) __attribute__((always_inline)) {
    const int t0 = tile * kKeys;
    const int wt0 = t0 + wrow;  // first key of this wave's half
    if constexpr (paged) {
      // The block ids of the tile's halves: with 16-token blocks two adjacent
      // table entries (one 8-byte scalar load unless the first is the row's
      // last entry, whose second half then lies past the context), else one
      // block holds both halves. t0 < kv_end, so entry e0 is in the row.
      const ConstI32* ctab = (const ConstI32*)(trow);
      const int e0 = t0 >> a.log2_block;
      int id0, id1;
      if (pair_ids && e0 + 1 < a.t_width) {
        typedef int32_t int2v __attribute__((ext_vector_type(2)));
        using ConstI32x2 = __attribute__((address_space(4))) const int2v;
        const int2v both = *(const ConstI32x2*)(ctab + e0);
        id0 = both.x;
        id1 = both.y;
      } else {
        id0 = ctab[e0];
        id1 = id0;
      }
      const uint32_t nb = static_cast<uint32_t>(a.num_blocks);
      const int mask = (static_cast<uint32_t>(id0) < nb ? 1 : 0) |
                       (static_cast<uint32_t>(id1) < nb ? 2 : 0);
      // An invalid id reads block 0; keys past the range read later rows of
      // the half's block (or of the first half's block when the second half
      // lies past the row): masked in the scores and zeroed in V before use.
      const int wid = wave_half ? id1 : id0;
      const int widc = static_cast<uint32_t>(wid) < nb ? wid : 0;
      if constexpr (A32) {
        const uint32_t soff = static_cast<uint32_t>(widc) * bs_bytes +
                              static_cast<uint32_t>(wt0 & (a.block_size - 1)) * ts_bytes;
        lds_load16_buf(rsrc_k, soff, off_k[0], kbuf + k_lds);
        lds_load16_buf(rsrc_k, soff, off_k[1], kbuf + k_lds + 4 * 16 * 8);
        lds_load16x2_buf(rsrc_v, soff, off_v[0], off_v[1] - 1024u, vbuf + v_lds);
      } else {
        const int64_t wbase = static_cast<int64_t>(widc) * a.c_bs +
                              (wt0 & (a.block_size - 1)) * a.c_ts + head_off;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          lds_load16_sbase(kc + wbase, off_k[j], kbuf + k_lds + j * 4 * 16 * 8);
          lds_load16_sbase(vc + wbase, off_v[j], vbuf + v_lds + j * 4 * kD);
        }
      }
      return mask;
    }
    // Contiguous K/V: keys past the range read the last row in range
    // instead (their scores are masked).
    if constexpr (A32) {
      // Lane offsets from the head's base.
      const int rk = min(wt0 + kkey, kv_end - 1) + static_cast<int>(krow0);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int rv = min(t0 + v_key[j], kv_end - 1) + static_cast<int>(krow0);
        lds_load16_sbase(kc + head_off, static_cast<uint32_t>(rk * c_ts + k_ch[j] * 8) * 2u,
                         kbuf + k_lds + j * 4 * 16 * 8);
        lds_load16_sbase(vc + head_off, static_cast<uint32_t>(rv * c_ts + v_ch[j] * 8) * 2u,
                         vbuf + v_lds + j * 4 * kD);
      }
    } else {
      // The same from the tile's first row (64-bit scalar base; a row within
      // the tile times c_ts < 2^26 stays below 2^32 bytes).
      const int64_t tbase = (krow0 + t0) * a.c_ts + head_off;
      const int rk = min(wt0 + kkey, kv_end - 1) - t0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int rv = min(t0 + v_key[j], kv_end - 1) - t0;
        lds_load16_sbase(kc + tbase, static_cast<uint32_t>(rk * c_ts + k_ch[j] * 8) * 2u,
                         kbuf + k_lds + j * 4 * 16 * 8);
        lds_load16_sbase(vc + tbase, static_cast<uint32_t>(rv * c_ts + v_ch[j] * 8) * 2u,
                         vbuf + v_lds + j * 4 * kD);
      }
    }
    return 3;
  };

  // Per-lane LDS element offsets of the fragment reads.
  // K (A operand of S^T): lane reads key `col` (half col / 16, key col % 16
  // of it), logical chunk 2*ks + half: element (col/16)*2048 +
  // (2*ks + half)*128 + (col%16)*8 = k_rd0 + 256*ks.
  const int k_rd0 = (col / 16) * 16 * kD + half * 16 * 8 + (col % 16) * 8;
  // V^T (A operand of O^T), read transposed: lane (group gq = lane / 16,
  // s = lane % 16) supplies the 8-byte row of key 16c + 8j + (gq/2)*4 + s/4 at
  // dims db*32 + (gq%2)*16 + 4*(s%4); after the transpose, lane gets
  // V[16c + 8j + half*4 + k][db*32 + col] in element k.
  int v_rd[kD / 32];
  {
    const int gq = lane / 16, sl = lane % 16;
    const int vkey = (gq / 2) * 4 + sl / 4;  // row within each 8-key group
#pragma unroll
    for (int db = 0; db < kD / 32; ++db) {
      const int chunk = 4 * db + 2 * (gq % 2) + (sl % 4) / 2;
      v_rd[db] = vkey * kD + ((chunk ^ swz_v(vkey)) * 8) + 4 * (sl % 2);
    }
  }

  f32x16_t o[kD / 32];
#pragma unroll
  for (int db = 0; db < kD / 32; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  // Softmax state of this lane's row: running maximum m (log2 domain, the
  // same in both halves of the row), the raw-score threshold above which a
  // tile moves it, and the sum l of this lane's half of the row's weights
  // (the halves are added once, at the end).
  const float scale_log2 = a.scale_log2;
  const float inv_scale_log2 = 1.f / scale_log2;
  float m = -INFINITY, neg_m = 0.f, thr = -INFINITY, l = 0.f;

  // Scores of one 32-key tile from LDS buffer kbuf: S^T = K . Q^T, s[i] is
  // key (i/4)*8 + half*4 + i%4 of this lane's row. One accumulation chain: a
  // dependent MFMA takes its accumulator straight from the previous one, so
  // a chain issues as fast as independent MFMAs would.
  auto scores = [&](const R* kbuf) __attribute__((always_inline)) {
    f32x16_t s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks)
      s = M::mma(__builtin_bit_cast(vec8, load_pack<R, 8>(kbuf + k_rd0 + 256 * ks)), qf[ks], s);
    return s;
  };

  // The rest of a tile: mask, online softmax, O^T += V^T . P^T from vbuf.
  auto finish = [&](int tile, f32x16_t s, const R* vbuf, int mask) __attribute__((always_inline)) {
    // Mask (causal, past the workgroup's keys, invalid blocks) only where the
    // tile reaches one of those limits for some row of the wave; interior
    // tiles skip it. Rows past the request are left unmasked: their lanes'
    // states are never stored.
    const int t0 = tile * kKeys;
    const bool interior = tile < nint && mask == 3;
    if (!interior) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = (i / 4) * 8 + half * 4 + (i % 4);  // key / 16 == i / 8
        const int kpos = t0 + key;
        const bool ok = (kpos <= qpos) & (kpos < kv_end) & (((mask >> (i / 8)) & 1) != 0);
        s[i] = ok ? s[i] : -INFINITY;
      }
    }
    float smax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) smax = fmaxf(smax, s[i]);
    // Online softmax in the log2 domain on scaled scores s * c (c > 0, so the
    // maximum can be taken on raw scores). The running maximum m is moved --
    // and O and l rescaled -- only when some row's tile maximum exceeds it by
    // more than kRescaleSlack, a wave-uniform decision taken on each lane's
    // half of the row against thr = (m + kRescaleSlack) / c; otherwise
    // exponents stay below 2^kRescaleSlack and the normalisation by l at the
    // end is unchanged.
    if (__ballot(smax > thr) != 0) {
      const float rmax = fmaxf(smax, partner32(smax, lane)) * scale_log2;
      const float mnew = fmaxf(m, rmax);
      const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m - mnew);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
      m = mnew;
      neg_m = m == -INFINITY ? 0.f : -m;  // all scores masked so far: p = 0
      thr = (m + kRescaleSlack) * inv_scale_log2;
    }
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(s[i], scale_log2, neg_m));

    // P^T fragments: reduction slot j of 16-key chunk c is this lane's
    // p[8c + j], i.e. key 16c + (j/4)*8 + half*4 + j%4. The half-row sum is
    // taken over the rounded 16-bit values (the weights the MFMA applies),
    // two per dot2 instruction.
    vec8 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Pack<R, 8> pk;
#pragma unroll
      for (int j = 0; j < 8; ++j) pk.v[j] = to_raw<E>(p[8 * c + j]);
      pf[c] = __builtin_bit_cast(vec8, pk);
      const Pack<uint32_t, 4> w = __builtin_bit_cast(Pack<uint32_t, 4>, pk);
#pragma unroll
      for (int j = 0; j < 4; ++j) l = E::dot2(w.v[j], kOnes2<E>, l);
    }
    // O^T += V^T . P^T with the same key mapping on the A side: slots 0-3
    // of chunk c hold keys 16c + half*4 .. +3, slots 4-7 keys 16c + 8 +
    // half*4 .. +3 (two transposed reads, 8 keys apart).
#pragma unroll
    for (int db = 0; db < kD / 32; ++db) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const short4_t lo = read_tr(vbuf + v_rd[db] + (16 * c) * kD);
        const short4_t hi = read_tr(vbuf + v_rd[db] + (16 * c + 8) * kD);
        const short4_t both[2] = {lo, hi};
        o[db] = M::mma(__builtin_bit_cast(vec8, both), pf[c], o[db]);
      }
    }
  };

  // Pipeline over three LDS buffers, unrolled by three so that each buffer
  // has a fixed role and every LDS address is a register plus an immediate.
  // Step t: wait for this wave's loads of tile t, barrier (every wave's tile
  // t is in LDS and every wave is done with tile t - 1), compute tile t's
  // scores, issue tile t + 2 into the buffer tile t - 1 used, finish tile t.
  // The loop sits inside the prologue's branch so that every path into it
  // has passed the prologue (the compiler's wait insertion is static).
  auto wait_tile = [&](bool next_in_flight, int tile, int tmask, R* vbuf) __attribute__((always_inline)) {
    // vmcnt(4) leaves the next tile's four loads in flight; vmcnt(0) waits
    // for everything (s_waitcnt encoding: vmcnt in bits 3:0, expcnt 6:4 = 7
    // (no wait), lgkmcnt 11:8).
    // lgkmcnt(0): this wave's reads of the buffer about to be refilled have
    // returned. The barrier is a bare s_barrier: __syncthreads() would add a
    // release fence that waits for every load in flight.
    if (next_in_flight)
      __builtin_amdgcn_s_waitcnt(0x0074);
    else
      __builtin_amdgcn_s_waitcnt(0x0070);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // A tail tile (past kv_end) or a half with an invalid block id holds
    // whatever the cache holds there: weight 0, but 0 * NaN is NaN, so each
    // wave zeroes those of its own V rows before the barrier publishes the
    // tile (K needs nothing: its scores are replaced by -inf).
    if (tile >= nfull || tmask != 3) {
      const int t0 = tile * kKeys;
      const int row = wave * kRowsPerWave + lane / 8;
      if (t0 + row >= kv_end || !((tmask >> (row / 16)) & 1)) {
        R* dst = vbuf + row * kD + (lane % 8) * 16;
        store_pack<R, 8>(dst, zero_pack<R, 8>());
        store_pack<R, 8>(dst + 8, zero_pack<R, 8>());
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zeros are in LDS
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  static_assert(kRowsPerWave * kD * 2 == kWave * 32, "V-row zeroing: 32 bytes per lane");
  static_assert(kRowsPerWave / 4 * 2 == 4, "vmcnt above assumes four loads per wave per tile");
  if (ntiles > t_begin) {
    int mask0 = issue_tile(t_begin, s_k[0], s_v[0]);
    int mask1 = ntiles > t_begin + 1 ? issue_tile(t_begin + 1, s_k[1], s_v[1]) : 0;
    int mask2 = 0;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      Pack<R, 8> p = zero_pack<R, 8>();
      if (row_ok) p = load_pack<R, 8>(qrow + ks * 16 + half * 8);
      qf[ks] = __builtin_bit_cast(vec8, p);
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    // One step on buffer B (tile t in B, tile t + 2 into (B + 2) % 3).
    auto step = [&](auto buf, int t) __attribute__((always_inline)) {
      constexpr int B = decltype(buf)::value;
      constexpr int N = (B + 2) % 3;
      int& mcur = B == 0 ? mask0 : (B == 1 ? mask1 : mask2);
      int& mnext = N == 0 ? mask0 : (N == 1 ? mask1 : mask2);
      const int mc = mcur;
      wait_tile(t + 1 < ntiles, t, mc, s_v[B]);
      // The score MFMAs go first: tile t + 2's block-id load and its wait
      // then overlap with them.
      const f32x16_t sc = scores(s_k[B]);
      if (t + 2 < ntiles) mnext = issue_tile(t + 2, s_k[N], s_v[N]);
      finish(t, sc, s_v[B], mc);
    };
    // Whole triples in the loop (one exit, so the accumulators keep their
    // registers across it), then up to two more steps.
    int t = t_begin;
    for (; t + 3 <= ntiles; t += 3) {
      step(std::integral_constant<int, 0>(), t);
      step(std::integral_constant<int, 1>(), t + 1);
      step(std::integral_constant<int, 2>(), t + 2);
    }
    if (t < ntiles) step(std::integral_constant<int, 0>(), t);
    if (t + 1 < ntiles) step(std::integral_constant<int, 1>(), t + 1);
  }

  // o[db][i] = O^T[d = db*32 + (i/4)*8 + half*4 + i%4][row].
  if (nparts > 1) {
    // Partition of a split (row block, KV head): publish (m, l, o) unless
    // every other partition has already arrived; the last arrival merges
    // all partitions in partition order (its own from registers: the values
    // its slot would hold), so the result does not depend on which one
    // arrives last. Partial region of (slot, head, wave): o as [db*16 + i]
    // [lane] floats, (m, l) as [2][lane].
    int32_t* ctr = a.counters + static_cast<int64_t>(counter) * a.num_kv_heads + head;
    auto region = [&](int p) {
      return (static_cast<int64_t>(slot + p) * a.num_kv_heads + head) * kWaves + wave;
    };
    if (tid == 0)
      s_arrived = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const bool last_now = s_arrived == nparts - 1;
    __syncthreads();  // s_arrived is written again below
    if (!last_now) {
      const int64_t r = region(part);
      float* acc = a.ws_acc + r * (kD / 32 * 16 * kWave) + lane;
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) store_coherent(acc + (db * 16 + i) * kWave, o[db][i]);
      store_coherent(a.ws_ml + r * 2 * kWave + lane, m);
      store_coherent(a.ws_ml + r * 2 * kWave + kWave + lane, l);
      wait_stores();
      __syncthreads();  // every wave's partial is at the coherent level
      if (tid == 0)
        s_arrived = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      if (s_arrived != nparts - 1) return;  // uniform
    }
    // Merge: mx = max m_p; o = sum_p 2^(m_p - mx) o_p, l likewise (m_p =
    // -inf: nothing of that partition is visible to the row, weight 0), in
    // partition order, the loads of kMergeBatch partitions in flight at once.
    float f[kMaxParts], lsum = 0.f, mx = -INFINITY;
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      f[p] = -INFINITY;
      if (p < nparts) f[p] = p == part ? m : load_coherent(a.ws_ml + region(p) * 2 * kWave + lane);
    }
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) mx = fmaxf(mx, f[p]);
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      f[p] = f[p] == -INFINITY ? 0.f : fast_exp2(f[p] - mx);
      if (p < nparts)
        lsum = fmaf(f[p], p == part ? l : load_coherent(a.ws_ml + region(p) * 2 * kWave + kWave + lane),
                    lsum);
    }
#pragma unroll
    for (int db = 0; db < kD / 32; ++db) {
      f32x16_t acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
      for (int p0 = 0; p0 < kMaxParts; p0 += kMergeBatch) {
        if (p0 >= nparts) break;
        float v[kMergeBatch][16];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          const int p = p0 + j;
          const float* src =
              a.ws_acc + region(p) * (kD / 32 * 16 * kWave) + db * 16 * kWave + lane;
#pragma unroll
          for (int i = 0; i < 16; ++i)
            v[j][i] = p < nparts && p != part ? load_coherent(src + i * kWave) : o[db][i];
        }
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[i] = fmaf(f[p0 + j], v[j][i], acc[i]);
      }
      o[db] = acc;
    }
    l = lsum;
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // The row's sum: both halves add (lane l & 31) + (lane l | 32).
  {
    const float other = partner32(l, lane);
    l = lane < 32 ? l + other : other + l;
  }
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

// Largest element offset a tile base computation can form, for the A32
// choice: the last row of the last block (paged) or up to a tile past the
// last row (contiguous: bases of a tile's rows past the end are formed, then
// replaced by the safe row), plus the other heads and a head row.
int64_t max_cache_offset(const AttnArgs& a) {
  const int64_t rows = a.tables != nullptr
                           ? static_cast<int64_t>(a.num_blocks - 1) * a.c_bs +
                                 static_cast<int64_t>(a.block_size - 1) * a.c_ts
                           : static_cast<int64_t>(a.num_blocks + kKeys) * a.c_ts;
  return rows + static_cast<int64_t>(a.num_kv_heads - 1) * a.c_hs + a.head_dim;
}

// ---------------------------------------------------------------------------
// Launch plan. Without one, workgroup i takes the i-th (row block, KV head)
// in request order, each with all of its keys. The plan kernel, one
// workgroup launched ahead of the attention kernel, lists the items instead:
//  * largest first (a counting sort on key tiles): the launch starts with
//    the long items and ends with short ones, instead of ending with
//    whatever long block came last in request order;
//  * split along the keys only where the launch lacks parallelism: a CU
//    streams tiles as fast with two workgroups as with three, and one
//    workgroup alone runs at about 4/5 of that, so an item is cut into
//    contiguous tile ranges of about T = (launch tiles) / (2 x CUs) tiles
//    (at least kMinPartTiles, at most kMaxParts ranges), raised until the
//    ranges fit the workspace's partial slots. A launch with plenty of
//    items (T above its largest item) is not split at all.
// Single-row requests (never split) count ctx / kSingleRowDiv tiles: a
// single-row workgroup streams its context latency-bound, so it is placed
// as if it had more tiles than its work alone would say (the mixed 4120-row
// step: 111.1 us at 48, 113.3 at 96, 112.4 at 40; A/B on two boxes).
// ---------------------------------------------------------------------------
constexpr int kPlanThreads = 256;
constexpr int kPlanPer = 16;  // row blocks per plan thread (registers)
constexpr int kMaxPlanBlocks = kPlanThreads * kPlanPer;
constexpr int kMaxPlanReqs = 2048;
constexpr int kPlanBuckets = 2 * kPlanThreads;  // sizes >= 511 share the first
constexpr int kMinPartTiles = 16;
constexpr int kSplitSlots = 1024;  // partial slots (partition x KV head)
constexpr int kSingleRowDiv = 48;
constexpr int64_t kPlanHeader = 256;  // [0]: number of items

// Exclusive scan of one value per thread over the workgroup (wave scans on
// DPP shuffles, then the wave totals); also returns the total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += u;
  }
  if (lane == kWave - 1) s_wave[wave] = incl;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / kWave; ++w) {
    const int t = s_wave[w];
    before += w < wave ? t : 0;
    total += t;
  }
  __syncthreads();  // s_wave is reused by the next scan
  return before + incl - v;
}

__device__ __forceinline__ int block_sum(int v, int* s_wave) {
  int total;
  block_exclusive_scan(v, s_wave, total);
  return total;
}

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int num_seqs, int bm,
    int ctx_cap, int64_t kv_rows, int cus, int heads, int part_cap, int max_entries,
    PrefillItem* __restrict__ plan, int32_t* __restrict__ count, int32_t* __restrict__ counters,
    int num_counters) {
  __shared__ int s_qb[kMaxPlanReqs + 1];  // request -> first row block
  __shared__ int s_qlen[kMaxPlanReqs];
  __shared__ int s_ctx[kMaxPlanReqs];
  __shared__ int s_kvc[kMaxPlanReqs];     // contiguous K/V: rows the request can read
  __shared__ int s_hist[kPlanBuckets];    // bucket -> items, then -> next position
  __shared__ int s_wave[kPlanThreads / kWave];
  const int tid = threadIdx.x;
  for (int i = tid; i < num_counters; i += kPlanThreads) counters[i] = 0;
  for (int i = tid; i < kPlanBuckets; i += kPlanThreads) s_hist[i] = 0;
  for (int r = tid; r < num_seqs; r += kPlanThreads) {
    const int q0 = cu_q[r], q1 = cu_q[r + 1], k0 = cu_k[r], k1 = cu_k[r + 1];
    const int q_len = max(q1 - q0, 0);
    s_qlen[r] = q_len;
    s_ctx[r] = min(k1 - k0, ctx_cap);
    s_kvc[r] = kv_rows >= 0 ? static_cast<int>(min<int64_t>(max<int64_t>(kv_rows - k0, 0),
                                                            INT_MAX))
                            : INT_MAX;
    s_qb[r] = (q_len + bm - 1) / bm;
  }
  __syncthreads();
  // Row blocks per request -> first row block (each thread a run of requests).
  const int per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
  const int r0 = min(num_seqs, tid * per), r1 = min(num_seqs, r0 + per);
  int run = 0;
  for (int r = r0; r < r1; ++r) run += s_qb[r];
  int nqb;
  int first = block_exclusive_scan(run, s_wave, nqb);
  for (int r = r0; r < r1; ++r) {
    const int n = s_qb[r];
    s_qb[r] = first;
    first += n;
  }
  if (tid == 0) s_qb[num_seqs] = nqb;
  __syncthreads();
  nqb = min(nqb, min(max_entries, kMaxPlanBlocks));

  // This thread's row blocks q = tid + k * kPlanThreads: request, block,
  // key tiles (the attention kernel's kv_end) and work estimate.
  int req[kPlanPer], rb[kPlanPer], tiles[kPlanPer], units[kPlanPer];
  int work = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int q = tid + k * kPlanThreads;
    req[k] = -1;
    rb[k] = tiles[k] = units[k] = 0;
    if (q < nqb) {
      int lo = 0, hi = num_seqs - 1;  // last request whose first block <= q
      while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (s_qb[mid] <= q) lo = mid;
        else hi = mid - 1;
      }
      const int q_len = s_qlen[lo], ctx = s_ctx[lo];
      const int b = q - s_qb[lo];
      const int last = min(q_len, (b + 1) * bm) - 1;
      const int kv_end = max(0, min(min(ctx, ctx - q_len + last + 1), s_kvc[lo]));
      req[k] = lo;
      rb[k] = b;
      tiles[k] = (kv_end + kKeys - 1) / kKeys;
      const bool single = kv_rows < 0 && q_len == 1;
      units[k] = single ? (max(ctx, 0) + kSingleRowDiv - 1) / kSingleRowDiv : tiles[k];
      if (single) tiles[k] = -tiles[k] - 1;  // marks a single row (never split)
      work += units[k];
    }
  }
  const int64_t total = block_sum(work, s_wave);
  int target = static_cast<int>(max<int64_t>(
      kMinPartTiles, min<int64_t>((total * heads + 2 * cus - 1) / (2 * cus), INT_MAX / 4)));
  auto parts_of = [&](int t, int tgt) {
    return t > tgt ? min(kMaxParts, (t + tgt - 1) / tgt) : 1;
  };
  for (int iter = 0;; ++iter) {  // raise the target until the partitions fit
    int need = 0;
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) {
      const int n = parts_of(tiles[k], target);
      need += n > 1 ? n : 0;
    }
    if (block_sum(need, s_wave) <= part_cap) break;
    if (iter == 16) {
      target = INT_MAX / 4;  // no split
      break;
    }
    target *= 2;
  }
  // Part p of n covers tiles [p * tiles / n, (p + 1) * tiles / n).
  auto bucket_of = [](int size) { return kPlanBuckets - 1 - min(size, kPlanBuckets - 1); };
  int nsplit = 0, nslots = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    if (req[k] < 0) continue;
    const int n = parts_of(tiles[k], target);
    for (int p = 0; p < n; ++p) {
      const int size = n == 1 ? units[k] : (p + 1) * tiles[k] / n - p * tiles[k] / n;
      atomicAdd(&s_hist[bucket_of(size)], 1);
    }
    nsplit += n > 1;
    nslots += n > 1 ? n : 0;
  }
  // Split units and their partial slots, numbered in thread order.
  int units_total, slots_total;
  int unit = block_exclusive_scan(nsplit, s_wave, units_total);
  int slot = block_exclusive_scan(nslots, s_wave, slots_total);
  // Bucket start positions (largest sizes first): two buckets per thread.
  const int h0 = s_hist[2 * tid], h1 = s_hist[2 * tid + 1];
  int items;
  const int start = block_exclusive_scan(h0 + h1, s_wave, items);
  s_hist[2 * tid] = start;
  s_hist[2 * tid + 1] = start + h0;
  if (tid == 0) count[0] = min(items, max_entries);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    if (req[k] < 0) continue;
    const int t = tiles[k] < 0 ? -tiles[k] - 1 : tiles[k];
    const int n = parts_of(tiles[k], target);
    for (int p = 0; p < n; ++p) {
      const int begin = p * t / n, end = (p + 1) * t / n;
      const int pos = atomicAdd(&s_hist[bucket_of(n == 1 ? units[k] : end - begin)], 1);
      if (pos >= max_entries) continue;
      PrefillItem it;
      it.req = req[k];
      it.qblock = rb[k];
      it.tile_begin = begin;
      it.tile_end = end;
      it.part = p;
      it.nparts = n;
      it.slot = n > 1 ? slot : 0;
      it.counter = n > 1 ? unit : 0;
      plan[pos] = it;
    }
    if (n > 1) {
      slot += n;
      ++unit;
    }
  }
}

int part_cap_of(int32_t num_kv_heads) { return max(2, kSplitSlots / num_kv_heads); }

template <typename E, int G>
int32_t launch_g(const AttnArgs& a, hipStream_t stream) {
  constexpr int BM = kRows * kWaves / G;
  const int64_t blocks = a.prefill_plan != nullptr
                             ? a.max_entries
                             : (static_cast<int64_t>(a.num_rows) + BM - 1) / BM + a.num_seqs;
  const dim3 grid(static_cast<uint32_t>(blocks * a.num_kv_heads));
  const bool a32 = a.c_bs >= 0 && a.c_hs >= 0 && max_cache_offset(a) < (int64_t(1) << 31);
  const bool paged = a.tables != nullptr;
  if (a32 && paged)
    paged_prefill_mfma_kernel<E, G, true, true><<<grid, kThreads, 0, stream>>>(a);
  else if (a32)
    paged_prefill_mfma_kernel<E, G, true, false><<<grid, kThreads, 0, stream>>>(a);
  else if (paged)
    paged_prefill_mfma_kernel<E, G, false, true><<<grid, kThreads, 0, stream>>>(a);
  else
    paged_prefill_mfma_kernel<E, G, false, false><<<grid, kThreads, 0, stream>>>(a);
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
         (a.tables == nullptr || a.block_size >= 16) && a.c_ts >= kD &&
         a.c_ts < (int64_t(1) << 26);  // lane offsets (< 16 rows) stay in int32
}

int32_t launch_prefill_mfma(const AttnArgs& a, int32_t dtype, hipStream_t stream) {
  if (!prefill_mfma_supported(a, dtype)) return MI_ERR_UNSUPPORTED;
  return dtype == MI_DTYPE_BF16 ? launch_typed<BF16>(a, stream) : launch_typed<F16>(a, stream);
}

int32_t prefill_counters(int32_t num_kv_heads) {
  // At most part_cap / 2 split (row block, KV head)s per KV head.
  return part_cap_of(num_kv_heads) / 2 * num_kv_heads;
}

namespace {
// Workspace: [count][counters][plan][ml partials][o partials], each region
// 256-byte aligned. The plan kernel zeroes the counters, so the workspace
// needs no initialisation.
struct PrefillLayout {
  int64_t max_entries, counters_off, plan_off, ml_off, acc_off, total;
};
PrefillLayout prefill_layout(int32_t num_rows, int32_t num_seqs, int32_t group,
                             int32_t num_kv_heads) {
  auto round256 = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int bm = kRows * kWaves / group;
  const int64_t regions = static_cast<int64_t>(part_cap_of(num_kv_heads)) * num_kv_heads * kWaves;
  PrefillLayout l;
  l.max_entries = (static_cast<int64_t>(num_rows) + bm - 1) / bm + num_seqs +
                  part_cap_of(num_kv_heads);
  l.counters_off = kPlanHeader;
  l.plan_off = l.counters_off + round256(int64_t(prefill_counters(num_kv_heads)) * 4);
  l.ml_off = l.plan_off + round256(l.max_entries * static_cast<int64_t>(sizeof(PrefillItem)));
  l.acc_off = l.ml_off + round256(regions * 2 * kWave * 4);
  l.total = l.acc_off + regions * (kD / 32) * 16 * kWave * 4;
  return l;
}
}  // namespace

int64_t prefill_workspace_bytes(int32_t num_rows, int32_t num_seqs, int32_t group,
                                int32_t num_kv_heads) {
  if (num_rows <= 0 || num_seqs <= 0 || num_seqs > kMaxPlanReqs || num_kv_heads <= 0 ||
      (group != 1 && group != 2 && group != 4))
    return 0;
  const int bm = kRows * kWaves / group;
  if ((static_cast<int64_t>(num_rows) + bm - 1) / bm + num_seqs > kMaxPlanBlocks) return 0;
  return prefill_layout(num_rows, num_seqs, group, num_kv_heads).total;
}

int32_t launch_prefill_plan(const AttnArgs& a, void* workspace, hipStream_t stream) {
  if (prefill_workspace_bytes(a.num_rows, a.num_seqs, a.group, a.num_kv_heads) == 0)
    return MI_ERR_UNSUPPORTED;
  const PrefillLayout l = prefill_layout(a.num_rows, a.num_seqs, a.group, a.num_kv_heads);
  char* ws = static_cast<char*>(workspace);
  const bool paged = a.tables != nullptr;
  prefill_plan_kernel<<<1, kPlanThreads, 0, stream>>>(
      a.cu_q, a.cu_k, a.num_seqs, kRows * kWaves / a.group,
      paged ? a.t_width * a.block_size : INT_MAX, paged ? int64_t(-1) : int64_t(a.num_blocks),
      device_cus(), a.num_kv_heads, part_cap_of(a.num_kv_heads),
      static_cast<int>(l.max_entries), reinterpret_cast<PrefillItem*>(ws + l.plan_off),
      reinterpret_cast<int32_t*>(ws), reinterpret_cast<int32_t*>(ws + l.counters_off),
      prefill_counters(a.num_kv_heads));
  return check_launch("paged prefill plan");
}

int32_t launch_prefill_mfma_planned(AttnArgs a, int32_t dtype, void* workspace, bool plan_ready,
                                    hipStream_t stream) {
  if (!prefill_mfma_supported(a, dtype) ||
      prefill_workspace_bytes(a.num_rows, a.num_seqs, a.group, a.num_kv_heads) == 0)
    return MI_ERR_UNSUPPORTED;
  if (!plan_ready) {
    const int32_t st = launch_prefill_plan(a, workspace, stream);
    if (st != MI_OK) return st;
  }
  const PrefillLayout l = prefill_layout(a.num_rows, a.num_seqs, a.group, a.num_kv_heads);
  char* ws = static_cast<char*>(workspace);
  a.prefill_plan = reinterpret_cast<PrefillItem*>(ws + l.plan_off);
  a.prefill_count = reinterpret_cast<int32_t*>(ws);
  a.max_entries = static_cast<int32_t>(l.max_entries);
  a.ws_ml = reinterpret_cast<float*>(ws + l.ml_off);
  a.ws_acc = reinterpret_cast<float*>(ws + l.acc_off);
  a.counters = reinterpret_cast<int32_t*>(ws + l.counters_off);
  return dtype == MI_DTYPE_BF16 ? launch_typed<BF16>(a, stream) : launch_typed<F16>(a, stream);
}

}  // namespace mi
