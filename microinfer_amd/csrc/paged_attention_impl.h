// Vector (non-MFMA) paged attention kernels for gfx950.
//
// Decode replaces _paged_decode_kernel / _paged_decode_reduce_kernel
// (microinfer/layer/triton_paged_attention.py:40-131, :236-257); varlen mode
// covers causal prefill rows for dtypes or shapes the MFMA kernel does not
// take, replacing the reference-path fallback (layer/paged_attention.py:22-67).
//
// Design:
//  * One wavefront = one work item (sequence, KV head, context partition).
//    All G = Hq/Hkv query heads of that KV head are processed together, so a
//    K/V row is fetched from HBM once per step instead of G times.
//  * A head row of D elements is spread over LPR lanes, VEC elements (16 B)
//    per lane, so one load instruction fetches PPW = 64/LPR whole rows; a tile
//    issues UNROLL such K loads and UNROLL V loads before any arithmetic.
//  * Scores: per-lane partial dot products, xor-reduced over the LPR lanes of
//    a row. Online softmax runs in the log2 domain (q is pre-scaled by
//    scale*log2 e) with a wave-uniform running max, so the running sum and the
//    P.V accumulator stay per-lane partials until one final cross-lane merge.
//  * Partitions are planned on the device from context_lens: every wave
//    recomputes the same prefix sum over sequences, so the launch shape
//    depends only on the batch size and stays valid under hipGraph replay.
#pragma once

#include "paged_attention.h"

namespace mi {

struct WorkItem {
  int seq, part, nparts, blk_begin, blk_end, ctx;
};

// Decode plan, computed identically by every wave of a launch.
//  nb_r  = ceil(min(ctx_r, width * B) / B) blocks of sequence r
//  PB    = adaptive: max(min_part_blocks, ceil(sum nb * Hkv / target_items))
//          forced:   ceil(nb_r / min(split_k, nb_r)) per sequence
//  parts_r = max(1, ceil(nb_r / PB)); items are numbered sequence-major.
// Finds the item with index `key` (by_seq = false) or the first item of
// sequence `key` (by_seq = true). Returns false when no such item exists.
__device__ __forceinline__ bool decode_plan(const AttnArgs& a, int key, bool by_seq, int lane,
                                            WorkItem& it) {
  const int B = a.block_size;
  const int lb = a.log2_block;
  const int max_ctx = a.t_width * B;
  int pb_global = 1;
  if (a.split_k == 0) {
    int total = 0;
    for (int base = 0; base < a.num_seqs; base += kWave) {
      const int r = base + lane;
      if (r < a.num_seqs) {
        const int c = min(max(a.ctx[r], 0), max_ctx);
        total += (c + B - 1) >> lb;
      }
    }
    total = wave_sum_int(total);
    const int64_t want = static_cast<int64_t>(total) * a.num_kv_heads;
    const int pb = static_cast<int>((want + a.target_items - 1) / a.target_items);
    pb_global = max(a.min_part_blocks, max(pb, 1));
  }
  int running = 0;
  for (int base = 0; base < a.num_seqs; base += kWave) {
    const int r = base + lane;
    int c = 0, nb = 0, pb = 1, np = 0;
    if (r < a.num_seqs) {
      c = min(max(a.ctx[r], 0), max_ctx);
      nb = (c + B - 1) >> lb;
      if (a.split_k == 0) {
        pb = pb_global;
      } else {
        const int k = min(a.split_k, max(nb, 1));
        pb = max(1, (nb + k - 1) / k);
      }
      np = max(1, (nb + pb - 1) / pb);
    }
    const int incl = wave_inclusive_scan(np, lane);
    const int start = running + incl - np;
    const bool mine = (r < a.num_seqs) &&
                      (by_seq ? (r == key) : (key >= start && key < start + np));
    const uint64_t hit = __ballot(mine);
    if (hit) {
      const int src = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      const int first = __shfl(start, src, kWave);
      const int pbs = __shfl(pb, src, kWave);
      const int nbs = __shfl(nb, src, kWave);
      it.seq = __shfl(r, src, kWave);
      it.nparts = __shfl(np, src, kWave);
      it.ctx = __shfl(c, src, kWave);
      it.part = by_seq ? first : key - first;  // by_seq: first item index
      const int p = by_seq ? 0 : it.part;
      it.blk_begin = p * pbs;
      it.blk_end = min(nbs, it.blk_begin + pbs);
      return true;
    }
    running += __shfl(incl, kWave - 1, kWave);
  }
  return false;
}

template <typename E, int VEC, int LPR, int GMAX, bool EXACT, int UNROLL>
__global__ __launch_bounds__(kWave) void paged_attention_vector_kernel(const AttnArgs a) {
  using R = typename E::raw;
  constexpr int PPW = kWave / LPR;  // rows per load instruction
  constexpr int TILE = PPW * UNROLL;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int sub = lane % LPR;
  const int d0 = sub * VEC;
  const int head = blockIdx.y;
  const int w = blockIdx.x;
  const int G = EXACT ? GMAX : a.group;

  int seq, q_row, ctx, blk_begin, blk_end, nparts;
  if (a.varlen) {
    q_row = w;
    int lo = 0, hi = a.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.cu_q[mid] <= q_row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    const int q_len = a.cu_q[lo + 1] - a.cu_q[lo];
    const int c = a.cu_k[lo + 1] - a.cu_k[lo];
    ctx = c - q_len + (q_row - a.cu_q[lo]) + 1;
    if (a.tables != nullptr) ctx = min(ctx, a.t_width * a.block_size);
    ctx = max(ctx, 0);
    blk_begin = 0;
    blk_end = (ctx + a.block_size - 1) >> a.log2_block;
    nparts = 1;
  } else {
    WorkItem it;
    if (!decode_plan(a, w, false, lane, it)) return;
    // The plan is identical on every lane; keep it in scalar registers.
    seq = __builtin_amdgcn_readfirstlane(it.seq);
    q_row = seq;
    ctx = __builtin_amdgcn_readfirstlane(it.ctx);
    blk_begin = __builtin_amdgcn_readfirstlane(it.blk_begin);
    blk_end = __builtin_amdgcn_readfirstlane(it.blk_end);
    nparts = __builtin_amdgcn_readfirstlane(it.nparts);
  }

  // Query rows of the G heads, pre-scaled into the log2 domain.
  const R* qbase = static_cast<const R*>(a.q) + q_row * a.q_ts + d0;
  float qf[GMAX][VEC];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (EXACT || g < G) {
      const Pack<R, VEC> qp = load_pack<R, VEC>(qbase + (head * G + g) * a.q_hs);
#pragma unroll
      for (int j = 0; j < VEC; ++j) qf[g][j] = E::load(qp.v[j]) * a.scale_log2;
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) qf[g][j] = 0.f;
    }
  }

  float m[GMAX], lsum[GMAX], acc[GMAX][VEC];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    m[g] = -INFINITY;
    lsum[g] = 0.f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[g][j] = 0.f;
  }

  const R* kc = static_cast<const R*>(a.kc);
  const R* vc = static_cast<const R*>(a.vc);
  // Contiguous mode (varlen only, no block table): request `seq` owns K/V rows
  // cu_k[seq] .. cu_k[seq + 1] - 1 of a [rows, Hkv, D] array; num_blocks holds
  // the row count. It runs as one "block" that spans the whole request.
  const bool paged = a.tables != nullptr;
  const int32_t* trow = paged ? a.tables + seq * a.t_stride : nullptr;
  const int64_t row0 = paged ? 0 : a.cu_k[seq];
  const int lb = paged ? a.log2_block : 30;
  const int bmask = paged ? a.block_size - 1 : (1 << 30) - 1;
  const int64_t base_off = head * a.c_hs + d0 + row0 * a.c_ts;
  // Any in-bounds address; masked rows load from here and are discarded.
  const int64_t safe_off = head * a.c_hs + d0;
  int pos_begin, pos_end;
  if (paged) {
    pos_begin = blk_begin << lb;
    pos_end = min(ctx, blk_end << lb);
  } else {
    pos_begin = 0;
    pos_end = static_cast<int>(min<int64_t>(ctx, max<int64_t>(a.num_blocks - row0, 0)));
    blk_end = 1;
  }
  // A load instruction covers PPW consecutive positions; when PPW <= B they
  // always share one block, so its id is wave-uniform and read with readlane.
  const bool uniform_ids = !paged || PPW <= a.block_size;

  // Block ids of up to 64 blocks live in registers (one per lane).
  for (int chunk = blk_begin; chunk < blk_end; chunk += kWave) {
    const int cpos_begin = paged ? max(pos_begin, chunk << lb) : pos_begin;
    const int cpos_end = paged ? min(pos_end, (chunk + kWave) << lb) : pos_end;
    if (cpos_begin >= cpos_end) break;
    int my_blk = 0;
    if (paged) {
      const int b = chunk + lane;
      my_blk = b < blk_end ? trow[b] : -1;
    }

    for (int t0 = cpos_begin; t0 < cpos_end; t0 += TILE) {
      int64_t off[UNROLL];
      bool ok[UNROLL];
      if (uniform_ids) {
        // Block address is scalar; each lane adds its row and column.
        const int64_t lane_off = grp * a.c_ts + base_off;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          const int p0 = t0 + u * PPW;
          const int blk = __builtin_amdgcn_readlane(my_blk, ((p0 >> lb) - chunk) & (kWave - 1));
          const bool blk_ok = blk >= 0 && blk < a.num_blocks;
          const int64_t block_off = blk * a.c_bs + (p0 & bmask) * a.c_ts;
          ok[u] = blk_ok && p0 + grp < cpos_end;
          off[u] = ok[u] ? block_off + lane_off : safe_off;
        }
      } else {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          const int pos = t0 + u * PPW + grp;
          const int blk = __shfl(my_blk, ((pos >> lb) - chunk) & (kWave - 1), kWave);
          ok[u] = pos < cpos_end && blk >= 0 && blk < a.num_blocks;
          off[u] = ok[u] ? blk * a.c_bs + (pos & bmask) * a.c_ts + base_off : safe_off;
        }
      }
      // Issue every K and V load of the tile before any arithmetic.
      Pack<R, VEC> kp[UNROLL], vp[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) kp[u] = load_pack<R, VEC>(kc + off[u]);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) vp[u] = load_pack<R, VEC>(vc + off[u]);

      // Scores of this lane group's UNROLL positions.
      float s[UNROLL][GMAX];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        float kf[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) kf[j] = E::load(kp[u].v[j]);
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          float dot = 0.f;
#pragma unroll
          for (int j = 0; j < VEC; ++j) dot = fmaf(qf[g][j], kf[j], dot);
          dot = group_sum<LPR>(dot);
          s[u][g] = ok[u] ? dot : -INFINITY;
        }
      }

      // Online softmax per lane group (each group is its own split; groups
      // are merged once at the end), then P.V.
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (!EXACT && g >= G) continue;
        float tmax = s[0][g];
#pragma unroll
        for (int u = 1; u < UNROLL; ++u) tmax = fmaxf(tmax, s[u][g]);
        const float mnew = fmaxf(m[g], tmax);
        const float alpha = (mnew == -INFINITY) ? 1.f : exp2f(m[g] - mnew);
        m[g] = mnew;
        lsum[g] *= alpha;
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[g][j] *= alpha;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          const float p = ok[u] ? exp2f(s[u][g] - mnew) : 0.f;
          lsum[g] += p;
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[g][j] = fmaf(p, E::load(vp[u].v[j]), acc[g][j]);
        }
      }
    }
  }

  // Merge the PPW lane-group states: rescale to the wave max, then sum.
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    const float mw = xor_max<LPR, kWave>(m[g]);
    const float f = (m[g] == -INFINITY) ? 0.f : exp2f(m[g] - mw);
    m[g] = mw;
    lsum[g] = xor_sum<LPR, kWave>(lsum[g] * f);
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[g][j] = xor_sum<LPR, kWave>(acc[g][j] * f);
  }

  if (nparts == 1) {
    if (grp == 0) {
      R* obase = static_cast<R*>(a.out) + q_row * a.o_ts + d0;
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (!EXACT && g >= G) continue;
        const float inv = lsum[g] > 0.f ? 1.f / lsum[g] : 0.f;
        Pack<R, VEC> o;
#pragma unroll
        for (int j = 0; j < VEC; ++j) o.v[j] = E::store(acc[g][j] * inv);
        store_pack<R, VEC>(obase + (head * G + g) * a.o_hs, o);
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (!EXACT && g >= G) continue;
      const int64_t idx = (static_cast<int64_t>(w) * a.num_kv_heads + head) * G + g;
      if (grp == 0) {
        Pack<float, VEC> o;
#pragma unroll
        for (int j = 0; j < VEC; ++j) o.v[j] = acc[g][j];
        store_pack<float, VEC>(a.ws_acc + idx * a.head_dim + d0, o);
      }
      if (lane == 0) {
        a.ws_ml[idx * 2] = m[g];
        a.ws_ml[idx * 2 + 1] = lsum[g];
      }
    }
  }
}

// Merge the partition partials of each (sequence, KV head):
//   out = sum_i 2^(m_i - M) acc_i / sum_i 2^(m_i - M) l_i,  M = max_i m_i
// (the merge of microinfer/layer/triton_paged_attention.py:244-257, in the log2
// domain). Empty partitions (m = -inf) weigh zero.
template <typename E>
__global__ __launch_bounds__(kWave) void paged_decode_reduce_kernel(const AttnArgs a) {
  using R = typename E::raw;
  const int lane = threadIdx.x;
  const int head = blockIdx.y;
  WorkItem it;
  if (!decode_plan(a, blockIdx.x, true, lane, it)) return;
  if (it.nparts <= 1) return;
  const int first = it.part;
  const int G = a.group;
  const int D = a.head_dim;
  for (int g = 0; g < G; ++g) {
    float mx = -INFINITY;
    for (int i = lane; i < it.nparts; i += kWave) {
      const int64_t idx = (static_cast<int64_t>(first + i) * a.num_kv_heads + head) * G + g;
      mx = fmaxf(mx, a.ws_ml[idx * 2]);
    }
    mx = xor_max<1, kWave>(mx);
    float total = 0.f;
    for (int i = lane; i < it.nparts; i += kWave) {
      const int64_t idx = (static_cast<int64_t>(first + i) * a.num_kv_heads + head) * G + g;
      const float mi = a.ws_ml[idx * 2];
      const float wgt = (mi == -INFINITY) ? 0.f : exp2f(mi - mx);
      total += wgt * a.ws_ml[idx * 2 + 1];
    }
    total = xor_sum<1, kWave>(total);
    const float inv = total > 0.f ? 1.f / total : 0.f;
    R* obase = static_cast<R*>(a.out) + it.seq * a.o_ts + (head * G + g) * a.o_hs;
    for (int d = lane; d < D; d += kWave) {
      float num = 0.f;
      for (int i = 0; i < it.nparts; ++i) {
        const int64_t idx = (static_cast<int64_t>(first + i) * a.num_kv_heads + head) * G + g;
        const float mi = a.ws_ml[idx * 2];
        const float wgt = (mi == -INFINITY) ? 0.f : exp2f(mi - mx);
        num = fmaf(wgt, a.ws_acc[idx * D + d], num);
      }
      obase[d] = E::store(num * inv);
    }
  }
}

// Dispatch over head_dim and group size for one element type.
template <typename E>
int32_t launch_vector_typed(const AttnArgs& a, hipStream_t stream) {
  using R = typename E::raw;
  constexpr int kPackElems = 16 / sizeof(R);
  const int D = a.head_dim;
  const int G = a.group;
  const dim3 grid(a.varlen ? a.num_rows : a.max_items, a.num_kv_heads);
  bool launched = false;

#define MI_VEC_LAUNCH(DIM, GM, EX)                                                     \
  do {                                                                                  \
    constexpr int VEC_ = (DIM) < kPackElems ? (DIM) : kPackElems;                       \
    constexpr int LPR_ = (DIM) / VEC_;                                                  \
    paged_attention_vector_kernel<E, VEC_, LPR_, GM, EX, 8><<<grid, kWave, 0, stream>>>(a); \
    launched = true;                                                                    \
  } while (0)

#define MI_VEC_DIM(DIM)                                                                 \
  case DIM:                                                                             \
    if (G == 1) MI_VEC_LAUNCH(DIM, 1, true);                                            \
    else if (G == 2) MI_VEC_LAUNCH(DIM, 2, true);                                       \
    else if (G == 4) MI_VEC_LAUNCH(DIM, 4, true);                                       \
    else if (G == 8) MI_VEC_LAUNCH(DIM, 8, true);                                       \
    else if (G == 3 && (DIM) >= 64) MI_VEC_LAUNCH(DIM, 4, false);                       \
    else if (G < 8 && (DIM) >= 64) MI_VEC_LAUNCH(DIM, 8, false);                        \
    break;

  switch (D) {
    MI_VEC_DIM(2)
    MI_VEC_DIM(4)
    MI_VEC_DIM(8)
    MI_VEC_DIM(16)
    MI_VEC_DIM(32)
    MI_VEC_DIM(64)
    MI_VEC_DIM(128)
    MI_VEC_DIM(256)
    default:
      break;
  }
#undef MI_VEC_DIM
#undef MI_VEC_LAUNCH
  if (!launched)
    return fail(MI_ERR_UNSUPPORTED,
                "paged attention: no kernel for head_dim=" + std::to_string(D) +
                    " group=" + std::to_string(G));
  int32_t st = check_launch("paged attention");
  if (st != MI_OK) return st;
  if (!a.varlen && a.split_k != 1) {
    const dim3 rgrid(a.num_seqs, a.num_kv_heads);
    paged_decode_reduce_kernel<E><<<rgrid, kWave, 0, stream>>>(a);
    st = check_launch("paged decode reduce");
  }
  return st;
}

}  // namespace mi
