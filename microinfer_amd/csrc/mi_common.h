// Shared device helpers for the gfx950 paged-KV kernels: element types,
// 16-byte vector packs and 64-lane wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "mi_attn.h"

namespace mi {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------------------
// Element types. 16-bit floats travel as raw uint16_t bit patterns; all
// arithmetic is float32.
// ---------------------------------------------------------------------------
struct F32 {
  using raw = float;
  static __device__ __forceinline__ float load(raw x) { return x; }
  static __device__ __forceinline__ raw store(float x) { return x; }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct BF16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float load(raw x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  // a.lo*b.lo + a.hi*b.hi + c on two packed elements (v_dot2_f32_bf16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                          __builtin_bit_cast(bf16x2_t, b), c, false);
  }
  // Round to nearest even; NaN becomes the canonical quiet NaN 0x7FC0.
  static __device__ __forceinline__ raw store(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<raw>(u >> 16);
  }
};

struct F16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float load(raw x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  // a.lo*b.lo + a.hi*b.hi + c on two packed elements (v_dot2_f32_f16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
  }
  static __device__ __forceinline__ raw store(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

// 2^x with the hardware v_exp_f32 (about 1 ulp; results below the normal
// range flush to zero, which only affects weights already < 2^-126).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// N consecutive raw elements moved with one load/store instruction.
template <typename R, int N>
struct alignas(sizeof(R) * N) Pack {
  R v[N];
};

template <typename R, int N>
__device__ __forceinline__ Pack<R, N> load_pack(const R* p) {
  return *reinterpret_cast<const Pack<R, N>*>(p);
}

template <typename R, int N>
__device__ __forceinline__ void store_pack(R* p, const Pack<R, N>& v) {
  *reinterpret_cast<Pack<R, N>*>(p) = v;
}

// Scheduling fence for loaded registers: an empty asm that "rewrites" every
// dword of the pack, so no instruction that uses the pack can be moved above
// this point. Double-buffered loops call it where a buffer starts being
// consumed, which keeps the compiler from waiting on the buffer that is
// still in flight.
template <typename R, int N>
__device__ __forceinline__ void pin(Pack<R, N>& p) {
  constexpr int W = sizeof(Pack<R, N>) / 4;
  static_assert(sizeof(Pack<R, N>) % 4 == 0, "pack must be whole dwords");
  Pack<uint32_t, W> w = __builtin_bit_cast(Pack<uint32_t, W>, p);
#pragma unroll
  for (int i = 0; i < W; ++i) asm volatile("" : "+v"(w.v[i]));
  p = __builtin_bit_cast(Pack<R, N>, w);
}

// Direct global->LDS load of 16 bytes per lane: lane i's bytes land at
// lds_dst + 16 i (global_load_lds_dwordx4, LDS base in M0; one wait state
// between the M0 write and the load). Issued as inline assembly so that the
// compiler does not track it: its own wait insertion would otherwise wait for
// these loads before every LDS read. The kernel waits for them explicitly
// (vmcnt) and orders them with bare barriers.
__device__ __forceinline__ void lds_load16(const void* src, const void* lds_dst) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) void*)(lds_dst)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// The same load with a scalar base and a per-lane 32-bit byte offset
// (saddr form), which saves the per-lane 64-bit address arithmetic.
__device__ __forceinline__ void lds_load16_sbase(const void* base, uint32_t byte_off,
                                                 const void* lds_dst) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) void*)(lds_dst)));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(byte_off), "s"(base), "s"(lds)
               : "memory", "m0");
}

template <typename R, int N>
__device__ __forceinline__ Pack<R, N> zero_pack() {
  Pack<R, N> z;
#pragma unroll
  for (int i = 0; i < N; ++i) z.v[i] = R(0);
  return z;
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off without whole-cache maintenance. Relaxed
// agent-scope atomic loads and stores compile to global_load/store with the
// sc1 bit, which is coherent across the per-XCD L2 caches; a release fence
// would instead write back and invalidate the entire L2 of every writer.
// A writer publishes with store_coherent, waits for its stores to complete
// (wait_stores), then signals with an agent-scope atomic; a reader that
// observed the signal reads with load_coherent.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void wait_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---------------------------------------------------------------------------
// Wavefront reductions (xor butterflies; every participating lane ends with
// the result).
// ---------------------------------------------------------------------------
template <int FROM, int TO>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
  for (int o = FROM; o < TO; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

template <int FROM, int TO>
__device__ __forceinline__ float xor_max(float v) {
#pragma unroll
  for (int o = FROM; o < TO; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// DPP lane move within a 16-lane row (bound_ctrl off: every source used here
// is a valid lane). CTRL values: 0xB1 quad_perm[1,0,3,2] (xor 1),
// 0x4E quad_perm[2,3,0,1] (xor 2), 0x141 row_half_mirror, 0x140 row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes; every lane of a group gets the sum.
// Groups of up to 16 lanes reduce with DPP (no LDS traffic).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_move<0xB1>(v);
  if constexpr (N >= 4) v += dpp_move<0x4E>(v);
  if constexpr (N >= 8) v += dpp_move<0x141>(v);
  if constexpr (N >= 16) v += dpp_move<0x140>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    int t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  return v;
}

__host__ __device__ constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v >> 1); }

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local, read through mi_last_error()).
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
int32_t fail(int32_t status, const std::string& msg);
int32_t check_launch(const char* what);

inline size_t dtype_size(int32_t dtype) { return dtype == MI_DTYPE_F32 ? 4 : 2; }

inline bool valid_dtype(int32_t dtype) {
  return dtype == MI_DTYPE_F32 || dtype == MI_DTYPE_F16 || dtype == MI_DTYPE_BF16;
}

}  // namespace mi
