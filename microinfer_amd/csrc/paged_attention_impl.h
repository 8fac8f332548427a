// Vector (non-MFMA) paged attention kernel for gfx950.
//
// Decode replaces _paged_decode_kernel + _paged_decode_reduce_kernel
// (microinfer/layer/triton_paged_attention.py:40-131, :236-257); varlen mode
// covers causal prefill rows for dtypes or shapes the MFMA kernel does not
// take, replacing the reference-path fallback (layer/paged_attention.py:22-67).
//
// Design:
//  * One wavefront = one work item (sequence, KV head, context partition).
//    All G = Hq/Hkv query heads of that KV head are processed together, so a
//    K/V row is fetched from HBM once per step instead of G times.
//  * A head row of D elements is spread over LPR lanes, VEC elements (16 B)
//    per lane, so one load instruction fetches PPW = 64/LPR whole rows. A tile
//    is UNROLL such K loads plus UNROLL V loads, and tiles are double-buffered
//    in registers: tile i+1 is in flight while tile i is computed.
//  * Scores: per-lane partial dot products summed over the LPR lanes of a row
//    with DPP. Each lane group (PPW of them per wave) keeps its own
//    online-softmax state in the log2 domain; the groups, then the waves of
//    a workgroup (through LDS), are merged once at the end.
//  * Decode work items come from a plan computed on the device from
//    context_lens (decode_plan.hip), so the launch shape depends only on the
//    batch size and stays valid under hipGraph replay.
//  * Partitions of one (sequence, KV head) are merged in the same launch: each
//    publishes (acc, m, l) with L2-coherent stores and bumps an arrival
//    counter; the last arrival merges and writes the output, then re-zeroes
//    the counter.
#pragma once

#include "paged_attention.h"

namespace mi {

// One double-buffer slot: UNROLL K and V packs plus a validity bit per load.
template <typename R, int VEC, int UNROLL>
struct KVTile {
  Pack<R, VEC> k[UNROLL];
  Pack<R, VEC> v[UNROLL];
  uint32_t ok;
};

template <typename E, int VEC, int LPR, int GMAX, bool EXACT, int UNROLL, bool FAST, int NW>
__global__ __launch_bounds__(kWave * NW, 2) void paged_attention_vector_kernel(const AttnArgs a) {
  using R = typename E::raw;
  using Tile = KVTile<R, VEC, UNROLL>;
  constexpr int D = VEC * LPR;
  constexpr int PPW = kWave / LPR;  // rows per load instruction
  constexpr int TILE = PPW * UNROLL;
  // readfirstlane tells the compiler the wave index is uniform, which keeps
  // tile positions and block-id lookups scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int grp = lane / LPR;
  const int sub = lane % LPR;
  const int d0 = sub * VEC;
  // Flattened grid: consecutive workgroups are the KV heads of one item.
  const int head = blockIdx.x % a.num_kv_heads;
  const int w = blockIdx.x / a.num_kv_heads;
  const int G = EXACT ? GMAX : a.group;

  int seq, q_row, ctx, blk_begin, blk_end, nparts, first_item = 0, part = 0;
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
    // Work item from the step's plan (one scalar load). Items are validated so
    // that a stale or foreign plan can give wrong attention but never an
    // out-of-bounds access.
    typedef int32_t int8v __attribute__((ext_vector_type(8)));
    using ConstItem = __attribute__((address_space(4))) const int8v;
    static_assert(sizeof(PlanItem) == sizeof(int8v), "plan item is eight int32");
    const PlanItem it = __builtin_bit_cast(PlanItem, ((ConstItem*)(a.plan))[w]);  // C cast: address space
    if (it.seq < 0 || it.seq >= a.num_seqs || it.nparts < 1 || it.part < 0 ||
        it.part >= it.nparts || it.first_item < 0 || it.first_item + it.nparts > a.max_items)
      return;  // unused slot (uniform across the workgroup)
    seq = it.seq;
    q_row = seq;
    ctx = min(max(it.ctx, 0), a.t_width * a.block_size);
    blk_begin = max(it.blk_begin, 0);
    blk_end = min(it.blk_end, a.t_width);
    nparts = it.nparts;
    first_item = it.first_item;
    part = it.part;
  }

  // Fused append (decode): the partition holding position ctx - 1 owns the
  // step's new K/V row of (seq, head). Its wave 0 stores the row into the
  // cache and attends to it from registers, so no load of that position is
  // ordered after the store. A sequence whose plan context disagrees with
  // context_lens (stale plan, or a context past the table) is not appended.
  bool append = false;
  int64_t append_off = -1;  // element offset of the cache row; -1: no valid block
  Pack<R, VEC> new_kp, new_vp;
  if (!a.varlen && a.new_k != nullptr && ctx >= 1) {
    const int last = (ctx - 1) >> a.log2_block;
    append = blk_begin <= last && last < blk_end && a.ctx[seq] == ctx;
    if (append && wave == 0) {
      const int blk = a.tables[seq * a.t_stride + last];
      if (blk >= 0 && blk < a.num_blocks)
        append_off = blk * a.c_bs + ((ctx - 1) & (a.block_size - 1)) * a.c_ts + head * a.c_hs;
      new_kp = load_pack<R, VEC>(static_cast<const R*>(a.new_k) + seq * a.nk_ts +
                                 head * a.nk_hs + d0);
      new_vp = load_pack<R, VEC>(static_cast<const R*>(a.new_v) + seq * a.nv_ts +
                                 head * a.nv_hs + d0);
    }
  }

  // Query rows of the G heads. 16-bit types keep raw element pairs for the
  // packed dot2 instructions; scores are scaled into the log2 domain after
  // the row sum.
  constexpr bool PAIRS = sizeof(R) == 2;
  constexpr int QW = PAIRS ? VEC / 2 : VEC;
  using QWord = typename std::conditional<PAIRS, uint32_t, float>::type;
  const R* qbase = static_cast<const R*>(a.q) + q_row * a.q_ts + d0;
  QWord qv[GMAX][QW];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    Pack<R, VEC> qp = zero_pack<R, VEC>();
    if (EXACT || g < G) qp = load_pack<R, VEC>(qbase + (head * G + g) * a.q_hs);
    const Pack<QWord, QW> words = __builtin_bit_cast(Pack<QWord, QW>, qp);
#pragma unroll
    for (int j = 0; j < QW; ++j) qv[g][j] = words.v[j];
  }
  const float scale_log2 = a.scale_log2;

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
  // Contiguous mode (general path, varlen only, no block table): request `seq`
  // owns K/V rows cu_k[seq] .. cu_k[seq + 1] - 1 of a [rows, Hkv, D] array;
  // num_blocks holds the row count. It runs as one "block" spanning the request.
  const bool paged = FAST || a.tables != nullptr;
  const int32_t* trow = paged ? a.tables + seq * a.t_stride : nullptr;
  const int64_t row0 = paged ? 0 : a.cu_k[seq];
  const int lb = paged ? a.log2_block : 30;
  const int bmask = paged ? a.block_size - 1 : (1 << 30) - 1;
  // Scalar part of a row address (block, row-in-block, head) + per-lane part
  // (row within the load group, column). Masked loads read row 0 of block 0.
  const int64_t head_off = head * a.c_hs + row0 * a.c_ts;
  const int64_t safe_head_off = head * a.c_hs;
  const int lane_off = grp * static_cast<int>(a.c_ts) + d0;
  int pos_begin, pos_end;
  if (paged) {
    pos_begin = blk_begin << lb;
    pos_end = min(append ? ctx - 1 : ctx, blk_end << lb);
  } else {
    pos_begin = 0;
    pos_end = static_cast<int>(min<int64_t>(ctx, max<int64_t>(a.num_blocks - row0, 0)));
    blk_end = 1;
  }
  const int last_blk = paged ? max(blk_end - 1, 0) : 0;
  // Fast path (host guarantees a table and PPW <= B): the PPW positions of a
  // load share one block, so its id is wave-uniform. Ids are fetched with
  // scalar loads (constant address space), which keeps the lookups off the
  // vector-memory counter that orders the in-flight K/V loads.
  using ConstI32 = __attribute__((address_space(4))) const int32_t;
  ConstI32* ctab = (ConstI32*)(trow);  // address-space conversion needs a C cast

  // Issue the K/V loads of the tile starting at t0 into slot T.
  auto issue = [&](Tile& T, int t0) {
    T.ok = 0;
    if constexpr (FAST) {
      int ids[UNROLL];  // all scalar id loads first, one wait, then the K/V loads
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) ids[u] = ctab[min((t0 + u * PPW) >> lb, last_blk)];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int p0 = t0 + u * PPW;
        const int blk = ids[u];
        const bool blk_ok = p0 < pos_end && blk >= 0 && blk < a.num_blocks;
        const bool lane_ok = blk_ok && p0 + grp < pos_end;
        const int64_t soff = blk_ok ? blk * a.c_bs + (p0 & bmask) * a.c_ts + head_off
                                    : safe_head_off;
        const int loff = lane_ok ? lane_off : d0;
        T.k[u] = load_pack<R, VEC>(kc + soff + loff);
        T.v[u] = load_pack<R, VEC>(vc + soff + loff);
        T.ok |= static_cast<uint32_t>(lane_ok) << u;
      }
    } else {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int pos = t0 + u * PPW + grp;
        const int blk = paged ? trow[min(pos >> lb, last_blk)] : 0;
        const bool ok = pos < pos_end && blk >= 0 && blk < a.num_blocks;
        const int64_t off = ok ? blk * a.c_bs + (pos & bmask) * a.c_ts + head_off + d0
                               : safe_head_off + d0;
        T.k[u] = load_pack<R, VEC>(kc + off);
        T.v[u] = load_pack<R, VEC>(vc + off);
        T.ok |= static_cast<uint32_t>(ok) << u;
      }
    }
  };

  // Online softmax + P.V over one loaded tile (this lane group's positions).
  auto consume = [&](Tile& T) {
    // Nothing that reads this tile may be scheduled before this point (in
    // particular not next to the loads of the other, still in-flight tile).
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      pin(T.k[u]);
      pin(T.v[u]);
    }
    float s[UNROLL][GMAX];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const Pack<QWord, QW> kw = __builtin_bit_cast(Pack<QWord, QW>, T.k[u]);
      const bool ok = (T.ok >> u) & 1u;
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < QW; ++j) {
          if constexpr (PAIRS) {
            dot = E::dot2(qv[g][j], kw.v[j], dot);
          } else {
            dot = fmaf(qv[g][j], kw.v[j], dot);
          }
        }
        dot = group_sum<LPR>(dot) * scale_log2;
        s[u][g] = ok ? dot : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (!EXACT && g >= G) continue;
      float tmax = s[0][g];
#pragma unroll
      for (int u = 1; u < UNROLL; ++u) tmax = fmaxf(tmax, s[u][g]);
      const float mnew = fmaxf(m[g], tmax);
      const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m[g] - mnew);
      m[g] = mnew;
      lsum[g] *= alpha;
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[g][j] *= alpha;
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const float p = ((T.ok >> u) & 1u) ? fast_exp2(s[u][g] - mnew) : 0.f;
        lsum[g] += p;
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[g][j] = fmaf(p, E::load(T.v[u].v[j]), acc[g][j]);
      }
    }
  };

  // Double-buffered tile loop. The NW waves interleave the partition's tiles
  // (wave k takes tiles k, k + NW, ...); tile i+1 is in flight while tile i is
  // used.
  // The next tile is issued unconditionally (past the end its loads hit the
  // safe row and are masked), so every path through the loop has the same
  // loads in flight and the wait counts stay exact.
  constexpr int STRIDE = TILE * NW;
  if (pos_begin + wave * TILE < pos_end) {
    Tile A, B;
    int t0 = pos_begin + wave * TILE;
    issue(A, t0);
    while (true) {
      const int t1 = t0 + STRIDE;
      issue(B, t1);
      consume(A);
      if (t1 >= pos_end) break;
      const int t2 = t1 + STRIDE;
      issue(A, t2);
      consume(B);
      if (t2 >= pos_end) break;
      t0 = t2;
    }
  }

  // The appended row: wave 0 stores it into the cache (lane group 0) and
  // folds it into lane group 0's softmax state. A row whose block id is
  // invalid is neither stored nor attended, as a skipped append would leave
  // that position masked.
  if (append && wave == 0) {
    const bool ok = grp == 0 && append_off >= 0;
    if (ok) {
      store_pack<R, VEC>(const_cast<R*>(kc) + append_off + d0, new_kp);
      store_pack<R, VEC>(const_cast<R*>(vc) + append_off + d0, new_vp);
    }
    const Pack<QWord, QW> kw = __builtin_bit_cast(Pack<QWord, QW>, new_kp);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < QW; ++j) {
        if constexpr (PAIRS) {
          dot = E::dot2(qv[g][j], kw.v[j], dot);
        } else {
          dot = fmaf(qv[g][j], kw.v[j], dot);
        }
      }
      dot = group_sum<LPR>(dot) * scale_log2;
      if (!ok || (!EXACT && g >= G)) continue;
      const float mnew = fmaxf(m[g], dot);
      const float alpha = (m[g] == -INFINITY) ? 0.f : fast_exp2(m[g] - mnew);
      const float p = fast_exp2(dot - mnew);
      m[g] = mnew;
      lsum[g] = fmaf(lsum[g], alpha, p);
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[g][j] = fmaf(acc[g][j], alpha, p * E::load(new_vp.v[j]));
    }
  }

  // Merge the PPW lane-group states of this wave: rescale to the wave max,
  // then sum across groups.
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    const float mw = xor_max<LPR, kWave>(m[g]);
    const float f = (m[g] == -INFINITY) ? 0.f : fast_exp2(m[g] - mw);
    m[g] = mw;
    lsum[g] = xor_sum<LPR, kWave>(lsum[g] * f);
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[g][j] = xor_sum<LPR, kWave>(acc[g][j] * f);
  }

  // Merge the NW wave states through LDS; wave 0 carries on alone.
  if constexpr (NW > 1) {
    __shared__ float s_acc[NW][GMAX][D];
    __shared__ float s_ml[NW][GMAX][2];
    if (grp == 0) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int j = 0; j < VEC; ++j) s_acc[wave][g][d0 + j] = acc[g][j];
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        s_ml[wave][g][0] = m[g];
        s_ml[wave][g][1] = lsum[g];
      }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float mx = s_ml[0][g][0];
#pragma unroll
      for (int k = 1; k < NW; ++k) mx = fmaxf(mx, s_ml[k][g][0]);
      float l = 0.f, o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[j] = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const float mk = s_ml[k][g][0];
        const float f = (mk == -INFINITY) ? 0.f : fast_exp2(mk - mx);
        l = fmaf(f, s_ml[k][g][1], l);
#pragma unroll
        for (int j = 0; j < VEC; ++j) o[j] = fmaf(f, s_acc[k][g][d0 + j], o[j]);
      }
      m[g] = mx;
      lsum[g] = l;
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[g][j] = o[j];
    }
  }

  R* obase = static_cast<R*>(a.out) + q_row * a.o_ts + d0;
  if (nparts == 1) {
    if (grp == 0) {
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
    return;
  }

  // Publish this partition's state, then count arrivals; the last workgroup
  // of the (sequence, KV head) merges every partition and writes the output.
  // Partials in the partition's slot (first_item + part; the plan may
  // dispatch items in any order): ws_acc[(slot*Hkv + head)*G + g][D],
  // ws_ml[...][2].
  {
    const int64_t base = (static_cast<int64_t>(first_item + part) * a.num_kv_heads + head) * G;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (!EXACT && g >= G) continue;
      if (grp == 0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          store_coherent(a.ws_acc + (base + g) * D + d0 + j, acc[g][j]);
      }
      if (lane == 0) {
        store_coherent(a.ws_ml + (base + g) * 2, m[g]);
        store_coherent(a.ws_ml + (base + g) * 2 + 1, lsum[g]);
      }
    }
  }
  wait_stores();  // partials have reached the coherent level before arrival
  int32_t* counter = a.counters + static_cast<int64_t>(seq) * a.num_kv_heads + head;
  int arrived = 0;
  if (lane == 0)
    arrived = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  arrived = __shfl(arrived, 0, kWave);
  if (arrived != nparts - 1) return;

  // Last arrival: out = sum_i 2^(m_i - M) acc_i / sum_i 2^(m_i - M) l_i,
  // M = max_i m_i (the merge of microinfer/layer/triton_paged_attention.py:
  // 244-257 in the log2 domain; empty partitions, m = -inf, weigh zero).
  auto item_row = [&](int part, int g) {
    return (static_cast<int64_t>(first_item + part) * a.num_kv_heads + head) * G + g;
  };
  // Pass 1: lane i reads partition i's maxima.
  float mx[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) mx[g] = -INFINITY;
  for (int i = lane; i < nparts; i += kWave) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (EXACT || g < G) mx[g] = fmaxf(mx[g], load_coherent(a.ws_ml + item_row(i, g) * 2));
  }
#pragma unroll
  for (int g = 0; g < GMAX; ++g) mx[g] = xor_max<1, kWave>(mx[g]);

  // Pass 2, per batch of 64 partitions: weights on lane i; lane group grp
  // then sums partitions grp, grp + PPW, ... of the batch for its columns,
  // DEPTH partitions at a time with all their loads issued before use.
  constexpr int DEPTH = (GMAX * VEC >= 64) ? 1 : 64 / (GMAX * VEC);
  float total[GMAX], num[GMAX][VEC];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    total[g] = 0.f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) num[g][j] = 0.f;
  }
  for (int base = 0; base < nparts; base += kWave) {
    const int i = base + lane;
    float wgt[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      wgt[g] = 0.f;
      if ((EXACT || g < G) && i < nparts) {
        const float mi = load_coherent(a.ws_ml + item_row(i, g) * 2);
        const float li = load_coherent(a.ws_ml + item_row(i, g) * 2 + 1);
        wgt[g] = (mi == -INFINITY) ? 0.f : fast_exp2(mi - mx[g]);
        total[g] = fmaf(wgt[g], li, total[g]);
      }
    }
    const int batch = min(kWave, nparts - base);
    for (int k0 = 0; k0 * PPW < batch; k0 += DEPTH) {
      float vals[DEPTH][GMAX][VEC];
      float wj[DEPTH][GMAX];
#pragma unroll
      for (int kk = 0; kk < DEPTH; ++kk) {
        const int j0 = grp + (k0 + kk) * PPW;
        const bool valid = j0 < batch;
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          wj[kk][g] = __shfl(wgt[g], j0 & (kWave - 1), kWave);
          const float* src = a.ws_acc + item_row(base + (valid ? j0 : 0), g) * D + d0;
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            vals[kk][g][j] = ((EXACT || g < G) && valid) ? load_coherent(src + j) : 0.f;
          if (!valid) wj[kk][g] = 0.f;
        }
      }
#pragma unroll
      for (int kk = 0; kk < DEPTH; ++kk)
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
#pragma unroll
          for (int j = 0; j < VEC; ++j) num[g][j] = fmaf(wj[kk][g], vals[kk][g][j], num[g][j]);
    }
  }
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (!EXACT && g >= G) continue;
    const float t = xor_sum<1, kWave>(total[g]);
    float out[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = xor_sum<LPR, kWave>(num[g][j]);
    if (grp == 0) {
      const float inv = t > 0.f ? 1.f / t : 0.f;
      Pack<R, VEC> o;
#pragma unroll
      for (int j = 0; j < VEC; ++j) o.v[j] = E::store(out[j] * inv);
      store_pack<R, VEC>(obase + (head * G + g) * a.o_hs, o);
    }
  }
  // Leave the counter zeroed for the next launch (all partitions arrived).
  if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads per tile (per K and per V). Larger GQA groups hold more accumulator
// registers, so they use shorter tiles to keep two waves per SIMD resident.
#ifndef MI_TILE_UNROLL_SMALL_GROUP
#define MI_TILE_UNROLL_SMALL_GROUP 4
#endif
#ifndef MI_TILE_UNROLL_LARGE_GROUP
#define MI_TILE_UNROLL_LARGE_GROUP 4
#endif
#ifndef MI_WAVES_PER_GROUP
#define MI_WAVES_PER_GROUP 8
#endif
// Waves per workgroup: they split one partition and merge through LDS.
constexpr int kWavesPerGroup = MI_WAVES_PER_GROUP;
// Decode launches with more (sequence, KV head) pairs than the device has
// CUs use half-width workgroups: at about 145 VGPRs a CU holds one 8-wave
// workgroup but three 4-wave ones, so such a grid runs in one round instead
// of two. (Qwen3-0.6B heads, 64 sequences of 140 tokens: 12.4 us per launch
// instead of 15.6; 32 sequences, one 8-wave group per CU, stays faster.)
constexpr int kNarrowWavesPerGroup = 4;

constexpr int tile_unroll(int gmax) {
  return gmax <= 2 ? MI_TILE_UNROLL_SMALL_GROUP : MI_TILE_UNROLL_LARGE_GROUP;
}

// Dispatch over head_dim and group size for one element type.
template <typename E>
int32_t launch_vector_typed(const AttnArgs& a, hipStream_t stream) {
  using R = typename E::raw;
  constexpr int kPackElems = 16 / sizeof(R);
  const int D = a.head_dim;
  const int G = a.group;
  const dim3 grid((a.varlen ? a.num_rows : a.max_items) * a.num_kv_heads);
  const bool narrow =
      !a.varlen && static_cast<int64_t>(a.num_seqs) * a.num_kv_heads > device_cus();
  bool launched = false;

#define MI_VEC_KERNEL(DIM, GM, EX, FAST_, NW_)                                          \
  paged_attention_vector_kernel<E, ((DIM) < kPackElems ? (DIM) : kPackElems),             \
                                (DIM) / ((DIM) < kPackElems ? (DIM) : kPackElems), GM, EX, \
                                tile_unroll(GM), FAST_, NW_><<<grid, kWave * (NW_), 0, stream>>>(a)
#define MI_VEC_LAUNCH(DIM, GM, EX)                                                     \
  do {                                                                                  \
    constexpr int LPR_ = (DIM) / ((DIM) < kPackElems ? (DIM) : kPackElems);             \
    const bool fast_ = a.tables != nullptr && kWave / LPR_ <= a.block_size;             \
    if (fast_ && narrow) MI_VEC_KERNEL(DIM, GM, EX, true, kNarrowWavesPerGroup);         \
    else if (fast_) MI_VEC_KERNEL(DIM, GM, EX, true, kWavesPerGroup);                    \
    else if (narrow) MI_VEC_KERNEL(DIM, GM, EX, false, kNarrowWavesPerGroup);            \
    else MI_VEC_KERNEL(DIM, GM, EX, false, kWavesPerGroup);                              \
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
#undef MI_VEC_KERNEL
  if (!launched)
    return fail(MI_ERR_UNSUPPORTED,
                "paged attention: no kernel for head_dim=" + std::to_string(D) +
                    " group=" + std::to_string(G));
  return check_launch("paged attention");
}

}  // namespace mi
