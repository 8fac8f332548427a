// Dense ops of the decoder layer around the paged attention path, for decode
// batches on gfx950 (entry points declared in include/mi_model.h).
//
//  * mi_linear: y = x . w^T for m <= 64 rows. At decode batch sizes the
//    product is bound by streaming w once from HBM. A workgroup owns 16 (or
//    32) output columns and every row; its waves split k. Per 32-wide k-step
//    a wave loads one 16-byte fragment of each of its 16 weight rows (the A
//    operand of v_mfma_f32_16x16x32, so the weights are used as stored) and
//    one per 16 rows of x (the B operand) and accumulates y^T tiles; eight
//    k-steps' loads are issued before their MFMAs. The waves' sums are added
//    through LDS in wave order, so results do not depend on timing.
//  * mi_rms_norm_residual: one wave per row, the row held in registers
//    between the sum of squares and the scaling.
//  * mi_silu_mul: one 16-byte vector of gate and of up per thread.
//  * mi_linear_swiglu: the gate/up projection with the SwiGLU gate in its
//    epilogue (each workgroup sums a gate and the matching up tile).
#include "mi_common.h"
#include "mi_model.h"

namespace mi {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename E>
struct LinMfma;
template <>
struct LinMfma<BF16> {
  using vec8 = bf16x8_t;
  static __device__ __forceinline__ f32x4_t mma(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct LinMfma<F16> {
  using vec8 = f16x8_t;
  static __device__ __forceinline__ f32x4_t mma(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// round(round(silu(g)) * u) on 16-bit inputs: the rounding steps of torch's
// F.silu(gate) * up.
template <typename E>
__device__ __forceinline__ uint16_t silu_mul_round(uint16_t g, uint16_t u) {
  const float x = E::load(g);
  const float act = E::load(E::store(x / (1.f + expf(-x))));
  return E::store(act * E::load(u));
}

constexpr int kLinStep = 32;   // k per MFMA
constexpr int kLinChunk = 8;   // k-steps whose loads are issued together
constexpr int kLinMaxRows = 64;

struct LinArgs {
  const void* x;
  int64_t xs;
  const void* w;
  int64_t ws;
  void* y;
  int64_t ys;
  int32_t m, n, k;
  int32_t row_tiles;  // RT launches: 16-row tiles of x, one per workgroup
  int32_t inter;      // GLU launches: rows [0, inter) of w are the gate, the rest up
};

// NW waves split k (wave w: a contiguous range of k-steps); NT 16-column
// tiles per workgroup; MT 16-row tiles of x (m <= 16 MT). The waves' float32
// sums meet in LDS and are added in wave order.
// RT: each workgroup takes one 16-row tile of x (MT = 1) instead of every
// row, so x is read once per column tile rather than once per row tile and
// column tile; the row tiles of a column tile get blockIdx values equal
// modulo 8 -- the same XCD, so they share its L2 -- and are dispatched
// together, so the weights still come from HBM about once.
// GLU: the SwiGLU gate of a gate/up projection in the epilogue. Tile 0 is
// gate columns n0 .. n0 + 15 (weight rows n0 + c), tile 1 the matching up
// columns (weight rows inter + n0 + c); the workgroup writes
// round(round(silu(gate)) * up) to columns n0 .. n0 + 15 of y, with gate and
// up first rounded to the element type as the plain projection stores them.
template <typename E, int NW, int NT, int MT, bool RT, bool GLU = false>
__global__ __launch_bounds__(NW * kWave) void linear_kernel(const LinArgs a) {
  using M = LinMfma<E>;
  using vec8 = typename M::vec8;
  using R = uint16_t;
  constexpr int kAcc = NT * MT * 4;  // float32 sums per lane
  __shared__ float s_acc[NW][kAcc][kWave];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int col = lane % 16;   // weight row (output column) / x row within a tile
  const int quad = lane / 16;  // 8-element group of the k-step
  static_assert(!RT || MT == 1, "row-tiled launches take one row tile");
  static_assert(!GLU || (NT == 2 && !RT), "GLU launches: gate and up tiles, every row");
  int n0 = blockIdx.x * (GLU ? 16 : 16 * NT), r0 = 0;
  if constexpr (RT) {
    const int xcd = blockIdx.x % 8;
    const int rest = blockIdx.x / 8;
    r0 = 16 * (rest % a.row_tiles);
    n0 = ((rest / a.row_tiles) * 8 + xcd) * (16 * NT);
  }
  const int total = a.k / kLinStep;
  const int per_wave = (total + NW - 1) / NW;
  const int s_begin = wave * per_wave;
  const int s_end = min(s_begin + per_wave, total);

  f32x4_t acc[NT][MT];
#pragma unroll
  for (int u = 0; u < NT; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[u][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const R* wrow[NT];
  bool wok[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    // n % 16 == 0: a tile's columns exist or none do.
    const int wr = GLU ? u * a.inter + n0 : n0 + 16 * u;
    wok[u] = GLU ? n0 < a.inter : wr < a.n;
    wrow[u] = static_cast<const R*>(a.w) +
              static_cast<int64_t>(wok[u] ? wr + col : 0) * a.ws + quad * 8;
  }
  const R* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int r = r0 + 16 * t + col;
    xok[t] = r < a.m;
    xrow[t] = static_cast<const R*>(a.x) + static_cast<int64_t>(xok[t] ? r : 0) * a.xs + quad * 8;
  }
  for (int s0 = s_begin; s0 < s_end; s0 += kLinChunk) {
    // Steps past the wave's range (a partial last chunk) get zero fragments
    // and still run their MFMAs, adding 0: no MFMA sits under a per-step
    // branch or exec mask (MFMA ignores EXEC).
    vec8 wf[kLinChunk][NT];
    vec8 xf[kLinChunk][MT];
#pragma unroll
    for (int j = 0; j < kLinChunk; ++j) {
      const bool step_ok = s0 + j < s_end;
      const int off = (s0 + j) * kLinStep;
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        Pack<R, 8> p = zero_pack<R, 8>();
        if (step_ok && wok[u]) p = load_pack<R, 8>(wrow[u] + off);
        wf[j][u] = __builtin_bit_cast(vec8, p);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        Pack<R, 8> p = zero_pack<R, 8>();
        if (step_ok && xok[t]) p = load_pack<R, 8>(xrow[t] + off);
        xf[j][t] = __builtin_bit_cast(vec8, p);
      }
    }
#pragma unroll
    for (int j = 0; j < kLinChunk; ++j)
#pragma unroll
      for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[u][t] = M::mma(wf[j][u], xf[j][t], acc[u][t]);
  }

  // acc[u][t][j] = y^T[n0 + 16 u + 4 quad + j][16 t + col]. Every wave but
  // the first hands its sums over through LDS; the first adds them in wave
  // order and stores.
  if (wave > 0) {
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) s_acc[wave][(u * MT + t) * 4 + j][lane] = acc[u][t][j];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int wv = 1; wv < NW; ++wv)
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[u][t][j] += s_acc[wv][(u * MT + t) * 4 + j][lane];
  R* y = static_cast<R*>(a.y);
  if constexpr (GLU) {
    if (!wok[0]) return;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = r0 + 16 * t + col;
      if (r < a.m) {
        Pack<R, 4> v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v.v[j] = silu_mul_round<E>(E::store(acc[0][t][j]), E::store(acc[1][t][j]));
        store_pack<R, 4>(y + static_cast<int64_t>(r) * a.ys + n0 + 4 * quad, v);
      }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    if (!wok[u]) continue;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = r0 + 16 * t + col;
      if (r < a.m) {
        Pack<R, 4> v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v.v[j] = E::store(acc[u][t][j]);
        store_pack<R, 4>(y + static_cast<int64_t>(r) * a.ys + n0 + 16 * u + 4 * quad, v);
      }
    }
  }
}

template <typename E, int NW, int NT>
void launch_linear_mt(LinArgs a, bool row_tiled, hipStream_t stream) {
  const int col_tiles = (a.n + 16 * NT - 1) / (16 * NT);
  const int row_tiles = (a.m + 15) / 16;
  if (row_tiled && row_tiles > 1) {
    a.row_tiles = row_tiles;
    const dim3 grid(static_cast<uint32_t>((col_tiles + 7) / 8 * 8 * row_tiles));
    linear_kernel<E, NW, NT, 1, true><<<grid, NW * kWave, 0, stream>>>(a);
    return;
  }
  const dim3 grid(static_cast<uint32_t>(col_tiles));
  switch (row_tiles) {
    case 1: linear_kernel<E, NW, NT, 1, false><<<grid, NW * kWave, 0, stream>>>(a); break;
    case 2: linear_kernel<E, NW, NT, 2, false><<<grid, NW * kWave, 0, stream>>>(a); break;
    case 3: linear_kernel<E, NW, NT, 3, false><<<grid, NW * kWave, 0, stream>>>(a); break;
    default: linear_kernel<E, NW, NT, 4, false><<<grid, NW * kWave, 0, stream>>>(a); break;
  }
}

// Workgroup shape, from hipGraph-replayed timings of the Qwen3-0.6B
// projections on MI355X (us per launch at 64 rows):
//  * up to 16 rows (one row tile): 16 columns per workgroup while that gives
//    at most a few workgroups per CU, else 32 (each x fragment then serves
//    two weight tiles); eight waves split k when the columns give fewer
//    workgroups than CUs;
//  * more rows, n <= 2048: row-tiled, 8 waves, 16 columns (output projection
//    6.1 against 11.9 with every row per workgroup; down projection 8.1
//    against 16.3);
//  * more rows, n <= 4096: row-tiled, 8 waves, 32 columns (QKV 8.1 against
//    8.6);
//  * more rows, wider: every row per workgroup, 4 waves, 32 columns (gate/up
//    10.4 against 12.0 row-tiled).
template <typename E>
int32_t launch_linear(const LinArgs& a, hipStream_t stream) {
  const int cus = device_cus();
  const int64_t tiles16 = a.n / 16;
  if (a.m <= 16) {
    if (tiles16 >= 8 * static_cast<int64_t>(cus))
      launch_linear_mt<E, 4, 2>(a, false, stream);
    else if (tiles16 >= cus)
      launch_linear_mt<E, 4, 1>(a, false, stream);
    else
      launch_linear_mt<E, 8, 1>(a, false, stream);
  } else if (a.n <= 2048) {
    launch_linear_mt<E, 8, 1>(a, true, stream);
  } else if (a.n <= 4096) {
    launch_linear_mt<E, 8, 2>(a, true, stream);
  } else {
    launch_linear_mt<E, 4, 2>(a, false, stream);
  }
  return check_launch("mi_linear");
}

// Gate/up projection with the SwiGLU gate: 4 waves (as the plain projection
// of that width, so gate and up are summed in the same order) over every row,
// one gate and one up tile per workgroup.
template <typename E>
int32_t launch_linear_glu(LinArgs a, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(a.inter / 16));
  switch ((a.m + 15) / 16) {
    case 1: linear_kernel<E, 4, 2, 1, false, true><<<grid, 4 * kWave, 0, stream>>>(a); break;
    case 2: linear_kernel<E, 4, 2, 2, false, true><<<grid, 4 * kWave, 0, stream>>>(a); break;
    case 3: linear_kernel<E, 4, 2, 3, false, true><<<grid, 4 * kWave, 0, stream>>>(a); break;
    default: linear_kernel<E, 4, 2, 4, false, true><<<grid, 4 * kWave, 0, stream>>>(a); break;
  }
  return check_launch("mi_linear_swiglu");
}

// ---------------------------------------------------------------------------
// RMSNorm with the residual sum.
// ---------------------------------------------------------------------------
constexpr int kRowsPerBlock = 4;  // one wave per row
constexpr int kNormMaxDim = 8192;

struct NormArgs {
  const void* x;
  int64_t xs;
  const void* res;
  int64_t rs;
  const void* weight;
  void* out;
  int64_t os;
  void* res_out;
  int64_t ros;
  int32_t rows, dim;
  float eps;
};

// CPL: 8-element chunks per lane (dim <= 512 CPL).
template <typename E, int CPL>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void rms_norm_residual_kernel(
    const NormArgs a) {
  using R = uint16_t;
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= a.rows) return;
  const int chunks = a.dim / 8;
  const R* x = static_cast<const R*>(a.x) + row * a.xs;
  const R* res = a.res != nullptr ? static_cast<const R*>(a.res) + row * a.rs : nullptr;
  R* res_out = a.res_out != nullptr ? static_cast<R*>(a.res_out) + row * a.ros : nullptr;
  const R* wt = static_cast<const R*>(a.weight);
  // Every load of the row (x, residual, weight) is issued before the first
  // use, so the row costs one memory round trip.
  Pack<R, 8> s[CPL], w[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + i * kWave;
    if (c < chunks) w[i] = load_pack<R, 8>(wt + c * 8);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + i * kWave;
    if (c < chunks) {
      s[i] = load_pack<R, 8>(x + c * 8);
      if (res != nullptr) {
        const Pack<R, 8> r = load_pack<R, 8>(res + c * 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) s[i].v[j] = E::store(E::load(s[i].v[j]) + E::load(r.v[j]));
        if (res_out != nullptr) store_pack<R, 8>(res_out + c * 8, s[i]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = E::load(s[i].v[j]);
        ss = fmaf(f, f, ss);
      }
    }
  }
  ss = xor_sum<1, kWave>(ss);
  const float inv = rsqrtf(ss / static_cast<float>(a.dim) + a.eps);
  R* out = static_cast<R*>(a.out) + row * a.os;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + i * kWave;
    if (c < chunks) {
      Pack<R, 8> o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float n = E::load(E::store(E::load(s[i].v[j]) * inv));
        o.v[j] = E::store(n * E::load(w[i].v[j]));
      }
      store_pack<R, 8>(out + c * 8, o);
    }
  }
}

template <typename E>
int32_t launch_norm(const NormArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>((a.rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(kRowsPerBlock * kWave);
  const int cpl = (a.dim / 8 + kWave - 1) / kWave;
  if (cpl <= 2)
    rms_norm_residual_kernel<E, 2><<<grid, block, 0, stream>>>(a);
  else if (cpl <= 4)
    rms_norm_residual_kernel<E, 4><<<grid, block, 0, stream>>>(a);
  else if (cpl <= 8)
    rms_norm_residual_kernel<E, 8><<<grid, block, 0, stream>>>(a);
  else
    rms_norm_residual_kernel<E, 16><<<grid, block, 0, stream>>>(a);
  return check_launch("mi_rms_norm_residual");
}

// ---------------------------------------------------------------------------
// SwiGLU gate.
// ---------------------------------------------------------------------------
constexpr int kSiluThreads = 256;

template <typename E>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_kernel(const uint16_t* gu, int64_t gs,
                                                                uint16_t* out, int64_t os,
                                                                int32_t rows, int32_t inter) {
  using R = uint16_t;
  const int per_row = inter / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kSiluThreads + threadIdx.x;
  if (idx >= static_cast<int64_t>(rows) * per_row) return;
  const int r = static_cast<int>(idx / per_row);
  const int c = static_cast<int>(idx % per_row) * 8;
  const Pack<R, 8> g = load_pack<R, 8>(gu + r * gs + c);
  const Pack<R, 8> u = load_pack<R, 8>(gu + r * gs + inter + c);
  Pack<R, 8> o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o.v[j] = silu_mul_round<E>(g.v[j], u.v[j]);
  store_pack<R, 8>(out + r * os + c, o);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool half_type(int32_t dtype) { return dtype == MI_DTYPE_BF16 || dtype == MI_DTYPE_F16; }

}  // namespace
}  // namespace mi

extern "C" int32_t mi_linear(const void* x, int64_t x_row_stride, const void* w,
                             int64_t w_row_stride, void* y, int64_t y_row_stride, int32_t m,
                             int32_t n, int32_t k, int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear: bad dtype");
  if (m < 0 || n <= 0 || k <= 0 || n % 16 || k % kLinStep)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_linear: need m >= 0, n a positive multiple of 16, k of 32");
  if (!half_type(dtype)) return fail(MI_ERR_UNSUPPORTED, "mi_linear: 16-bit types only");
  if (m > kLinMaxRows) return fail(MI_ERR_UNSUPPORTED, "mi_linear: m above 64");
  if (m == 0) return MI_OK;
  if (!x || !w || !y) return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear: null pointer");
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear: row strides below the row lengths");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || x_row_stride % 8 ||
      w_row_stride % 8 || y_row_stride % 8)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear: pointers and row strides must be 16-byte "
                                         "aligned");
  LinArgs a{};
  a.x = x;
  a.xs = x_row_stride;
  a.w = w;
  a.ws = w_row_stride;
  a.y = y;
  a.ys = y_row_stride;
  a.m = m;
  a.n = n;
  a.k = k;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MI_DTYPE_BF16 ? launch_linear<BF16>(a, s) : launch_linear<F16>(a, s);
}

extern "C" int32_t mi_rms_norm_residual(const void* x, int64_t x_row_stride,
                                        const void* residual, int64_t residual_row_stride,
                                        const void* weight, float eps, void* out,
                                        int64_t out_row_stride, void* residual_out,
                                        int64_t residual_out_row_stride, int32_t rows,
                                        int32_t dim, int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm_residual: bad dtype");
  if (rows < 0 || dim <= 0 || dim % 8)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_rms_norm_residual: need rows >= 0 and dim a positive multiple of 8");
  if (!half_type(dtype))
    return fail(MI_ERR_UNSUPPORTED, "mi_rms_norm_residual: 16-bit types only");
  if (dim > kNormMaxDim) return fail(MI_ERR_UNSUPPORTED, "mi_rms_norm_residual: dim above 8192");
  if (rows == 0) return MI_OK;
  if (!x || !weight || !out)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm_residual: null pointer");
  if (x_row_stride < dim || out_row_stride < dim ||
      (residual && residual_row_stride < dim) ||
      (residual && residual_out && residual_out_row_stride < dim))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm_residual: row strides below dim");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) ||
      (residual && !aligned16(residual)) || (residual_out && !aligned16(residual_out)) ||
      x_row_stride % 8 || out_row_stride % 8 || (residual && residual_row_stride % 8) ||
      (residual_out && residual_out_row_stride % 8))
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_rms_norm_residual: pointers and row strides must be 16-byte aligned");
  NormArgs a{};
  a.x = x;
  a.xs = x_row_stride;
  a.res = residual;
  a.rs = residual_row_stride;
  a.weight = weight;
  a.out = out;
  a.os = out_row_stride;
  a.res_out = residual ? residual_out : nullptr;
  a.ros = residual_out_row_stride;
  a.rows = rows;
  a.dim = dim;
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MI_DTYPE_BF16 ? launch_norm<BF16>(a, s) : launch_norm<F16>(a, s);
}

extern "C" int32_t mi_silu_mul(const void* gate_up, int64_t gate_up_row_stride, void* out,
                               int64_t out_row_stride, int32_t rows, int32_t inter,
                               int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_silu_mul: bad dtype");
  if (rows < 0 || inter <= 0 || inter % 8)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_silu_mul: need rows >= 0 and inter a positive multiple of 8");
  if (!half_type(dtype)) return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: 16-bit types only");
  if (rows == 0) return MI_OK;
  if (!gate_up || !out) return fail(MI_ERR_INVALID_ARGUMENT, "mi_silu_mul: null pointer");
  if (gate_up_row_stride < 2 * static_cast<int64_t>(inter) || out_row_stride < inter)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_silu_mul: row strides below the row lengths");
  if (!aligned16(gate_up) || !aligned16(out) || gate_up_row_stride % 8 || out_row_stride % 8)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_silu_mul: pointers and row strides must be 16-byte aligned");
  const int64_t threads = static_cast<int64_t>(rows) * (inter / 8);
  const int64_t blocks = (threads + kSiluThreads - 1) / kSiluThreads;
  if (blocks > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* gu = static_cast<const uint16_t*>(gate_up);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (dtype == MI_DTYPE_BF16)
    silu_mul_kernel<BF16><<<static_cast<uint32_t>(blocks), kSiluThreads, 0, s>>>(
        gu, gate_up_row_stride, o, out_row_stride, rows, inter);
  else
    silu_mul_kernel<F16><<<static_cast<uint32_t>(blocks), kSiluThreads, 0, s>>>(
        gu, gate_up_row_stride, o, out_row_stride, rows, inter);
  return check_launch("mi_silu_mul");
}

extern "C" int32_t mi_linear_swiglu(const void* x, int64_t x_row_stride, const void* w,
                                    int64_t w_row_stride, void* y, int64_t y_row_stride,
                                    int32_t m, int32_t inter, int32_t k, int32_t dtype,
                                    void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear_swiglu: bad dtype");
  if (m < 0 || inter <= 0 || k <= 0 || inter % 16 || k % kLinStep)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_linear_swiglu: need m >= 0, inter a positive multiple of 16, k of 32");
  if (!half_type(dtype)) return fail(MI_ERR_UNSUPPORTED, "mi_linear_swiglu: 16-bit types only");
  if (m > kLinMaxRows) return fail(MI_ERR_UNSUPPORTED, "mi_linear_swiglu: m above 64");
  if (m == 0) return MI_OK;
  if (!x || !w || !y) return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear_swiglu: null pointer");
  if (x_row_stride < k || w_row_stride < k || y_row_stride < inter)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_linear_swiglu: row strides below the row lengths");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || x_row_stride % 8 ||
      w_row_stride % 8 || y_row_stride % 8)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_linear_swiglu: pointers and row strides must be 16-byte aligned");
  LinArgs a{};
  a.x = x;
  a.xs = x_row_stride;
  a.w = w;
  a.ws = w_row_stride;
  a.y = y;
  a.ys = y_row_stride;
  a.m = m;
  a.n = 2 * inter;
  a.k = k;
  a.inter = inter;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MI_DTYPE_BF16 ? launch_linear_glu<BF16>(a, s) : launch_linear_glu<F16>(a, s);
}
