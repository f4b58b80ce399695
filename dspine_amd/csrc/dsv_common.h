// Shared device/host helpers of the gfx950 verification kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dspine_verify.h"

namespace dsv {

void set_error(const char* fmt, ...);

#define DSV_FAIL(code, ...)        \
  do {                             \
    ::dsv::set_error(__VA_ARGS__); \
    return (code);                 \
  } while (0)

#define DSV_CHECK_LAUNCH(what)                                                             \
  do {                                                                                     \
    hipError_t e_ = hipGetLastError();                                                     \
    if (e_ != hipSuccess)                                                                  \
      DSV_FAIL(DSV_ERR_LAUNCH, "%s: HIP launch failed: %s", (what), hipGetErrorString(e_)); \
  } while (0)

constexpr int WAVE = 64;
constexpr uint32_t NEG_INF_BF16_KEY = 0x007Fu;  // key16 of bf16 -inf (0xFF80)

// ---------------------------------------------------------------------------------------
// Device-coherent accesses: what one workgroup hands to another inside a launch.  The L2 of an
// XCD is not coherent with the others', so these are relaxed device-scope atomic accesses
// (global_store / global_load with sc1: written through to, and read from, the device's
// coherence point) -- no full-L2 writeback or invalidate.  A producer publishes with st_dev
// stores, waits for them to complete (publish_wait), then bumps a device-scope counter; the
// workgroup whose increment completes the count reads with ld_dev.
// ---------------------------------------------------------------------------------------
template <class T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's memory accesses have completed (s_waitcnt vmcnt(0); the other
// counters are left at their maxima: expcnt 7, lgkmcnt 15).  The compiler treats the wait as
// touching no memory, so compiler-only barriers on both sides keep the publishing stores before
// it and the counter's atomic after it (no instruction is emitted for them).
__device__ __forceinline__ void publish_wait() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------------------
// Order-preserving keys.  -0.0 is folded onto +0.0 so that equal values share one key, as
// torch's comparisons (sort, argmax) treat them as equal.  Larger value -> larger key.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_f32(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
// 16-bit key of a bf16 value given as raw bits.
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
  b &= 0xffffu;
  if (b == 0x8000u) b = 0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
__device__ __forceinline__ float bf16_key_to_f32(uint32_t k) {
  uint32_t b = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even float -> bf16 bits (what torch's copy into a bf16 tensor does).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// e^x for the running softmax sums: 2^(x*log2e) with the product error folded back in,
// about 1 ulp over the range that matters (|x| < 104).
__device__ __forceinline__ float exp_fast(float x) {
  const float L = 1.44269502162933349609375f;  // fp32(log2 e)
  const float Llo = 1.925963033500011e-08f;    // log2 e - L
  float t = x * L;
  float err = fmaf(x, L, -t);
  err = fmaf(x, Llo, err);
  float r = __builtin_amdgcn_exp2f(t);
  return fmaf(r, err * 0.693147180559945309f, r);
}

// ---------------------------------------------------------------------------------------
// Wave / block reductions (wave64).
// ---------------------------------------------------------------------------------------
// Lane moves through DPP (gfx9 controls): quad permutes, row shifts / mirrors, row broadcasts
// and the whole-wave shift.  They run in the VALU, not through the LDS crossbar.
enum : int {
  DPP_QUAD_XOR1 = 0xB1,        // quad_perm [1, 0, 3, 2]
  DPP_QUAD_XOR2 = 0x4E,        // quad_perm [2, 3, 0, 1]
  DPP_ROW_SHR1 = 0x111,
  DPP_ROW_SHR2 = 0x112,
  DPP_ROW_SHR4 = 0x114,
  DPP_ROW_SHR8 = 0x118,
  DPP_WAVE_SHR1 = 0x138,
  DPP_ROW_MIRROR = 0x140,
  DPP_ROW_HALF_MIRROR = 0x141,
  DPP_ROW_BCAST15 = 0x142,
  DPP_ROW_BCAST31 = 0x143,
};

// Lane value moved by CTRL.  Lanes of disabled rows (ROWS mask) keep `old`; lanes whose source
// lies outside the pattern's range read 0 with ZERO, else keep `old`.
template <int CTRL, int ROWS = 0xF, bool ZERO = false, typename T>
__device__ __forceinline__ T dpp(T old, T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                             CTRL, ROWS, 0xF, ZERO));
  } else {
    const uint64_t o = __builtin_bit_cast(uint64_t, old), x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)o, (int)(uint32_t)x, CTRL, ROWS, 0xF, ZERO);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(o >> 32), (int)(uint32_t)(x >> 32), CTRL,
                                                              ROWS, 0xF, ZERO);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// The value of lane L (uniform).
template <int L, typename T>
__device__ __forceinline__ T readlane(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), L));
  } else {
    const uint64_t x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, L);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), L);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// The value of lane l (l uniform across the wave).
template <typename T>
__device__ __forceinline__ T readlane_at(T v, int l) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  } else {
    const uint64_t x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// Reduction over the 64 lanes (every lane active), result in every lane: quads, half rows and
// rows through DPP, then the four row results in a fixed order.
template <typename T, class F>
__device__ __forceinline__ T wave_reduce(T v, F op) {
  v = op(v, dpp<DPP_QUAD_XOR1>(v, v));
  v = op(v, dpp<DPP_QUAD_XOR2>(v, v));
  v = op(v, dpp<DPP_ROW_HALF_MIRROR>(v, v));
  v = op(v, dpp<DPP_ROW_MIRROR>(v, v));
  return op(op(readlane<0>(v), readlane<16>(v)), op(readlane<32>(v), readlane<48>(v)));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return wave_reduce(v, [](T x, T y) { return x + y; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce(v, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  return wave_reduce(v, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  return wave_reduce(v, [](uint64_t x, uint64_t y) { return x < y ? x : y; });
}
__device__ __forceinline__ float wave_max_f32(float v) {
  return wave_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}
// Inclusive prefix sum over lanes 0..63 (every lane active): row scans by shifts, then the row
// totals carried into the rows above.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  v += dpp<DPP_ROW_SHR1, 0xF, true>(T(0), v);
  v += dpp<DPP_ROW_SHR2, 0xF, true>(T(0), v);
  v += dpp<DPP_ROW_SHR4, 0xF, true>(T(0), v);
  v += dpp<DPP_ROW_SHR8, 0xF, true>(T(0), v);
  v += dpp<DPP_ROW_BCAST15, 0xA>(T(0), v);
  v += dpp<DPP_ROW_BCAST31, 0xC>(T(0), v);
  return v;
}
// The value of the lane below (lane 0: `first`).
template <typename T>
__device__ __forceinline__ T wave_prev(T v, T first) {
  return dpp<DPP_WAVE_SHR1, 0xF, false>(first, v);
}

// Block-wide reductions over NW waves (the block size / 64, a compile-time constant so that
// the final loop over the per-wave partials is fully unrolled).
// Block-wide sum.  `scratch` holds NW entries; result broadcast to every thread.
template <int NW, typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  constexpr int nw = NW;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  T s = T(0);
  for (int i = 0; i < nw; ++i) s += scratch[i];  // fixed order: deterministic
  return s;
}

// Block-wide exclusive prefix over thread order (deterministic); also returns the total.
template <int NW, typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* scratch, T* total) {
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  constexpr int nw = NW;
  T incl = wave_incl_scan(v);
  __syncthreads();
  if (lane == WAVE - 1) scratch[wid] = incl;
  __syncthreads();
  T before = T(0), tot = T(0);
  for (int i = 0; i < nw; ++i) {
    if (i < wid) before += scratch[i];
    tot += scratch[i];
  }
  if (total) *total = tot;
  return before + incl - v;
}

template <int NW>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* scratch) {
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  constexpr int nw = NW;
  v = wave_max_u64(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  uint64_t m = 0;
  for (int i = 0; i < nw; ++i) m = scratch[i] > m ? scratch[i] : m;
  return m;
}
template <int NW>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* scratch) {
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  constexpr int nw = NW;
  v = wave_min_u64(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  uint64_t m = ~0ull;
  for (int i = 0; i < nw; ++i) m = scratch[i] < m ? scratch[i] : m;
  return m;
}

}  // namespace dsv
