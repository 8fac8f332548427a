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
  // Three K/V tile buffers (48 KiB per workgroup).
  __shared__ __attribute__((aligned(16))) R s_k[3][kTileElems];
  __shared__ __attribute__((aligned(16))) R s_v[3][kTileElems];

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
  constexpr bool paged = PAGED;  // block tables given (else contiguous K/V)
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
  if (ntiles > 0) {
    int mask0 = issue_tile(0, s_k[0], s_v[0]);
    int mask1 = ntiles > 1 ? issue_tile(1, s_k[1], s_v[1]) : 0;
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
    int t = 0;
    for (; t + 3 <= ntiles; t += 3) {
      step(std::integral_constant<int, 0>(), t);
      step(std::integral_constant<int, 1>(), t + 1);
      step(std::integral_constant<int, 2>(), t + 2);
    }
    if (t < ntiles) step(std::integral_constant<int, 0>(), t);
    if (t + 1 < ntiles) step(std::integral_constant<int, 1>(), t + 1);
  }

  // o[db][i] = O^T[d = db*32 + (i/4)*8 + half*4 + i%4][row].
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

template <typename E, int G>
int32_t launch_g(const AttnArgs& a, hipStream_t stream) {
  constexpr int BM = kRows * kWaves / G;
  const int64_t blocks = (static_cast<int64_t>(a.num_rows) + BM - 1) / BM + a.num_seqs;
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

}  // namespace mi
