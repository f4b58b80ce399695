// Error plumbing and the small kernels of the verification path.
#include <stdarg.h>
#include <stdio.h>

#include "dsv_common.h"

namespace dsv {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

// ---------------------------------------------------------------------------------------
// Seeded uniforms (sampling/random.py:22-68): 32-bit murmur3 of the four words
// (seed lo, seed hi, position, column + (stream << 16)), h0 = 0, length 16; u = (h>>8)*2^-24.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }
__device__ __forceinline__ uint32_t murmur_block(uint32_t h, uint32_t k) {
  k *= 0xCC9E2D51u;
  k = rotl32(k, 15);
  k *= 0x1B873593u;
  h ^= k;
  h = rotl32(h, 13);
  return h * 5u + 0xE6546B64u;
}
__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}

__global__ void k_uniforms(const int64_t* seeds, const void* positions, int pos64, int64_t n, int width,
                           int stream_id, float* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * width) return;
  const int64_t row = i / width;
  const uint32_t col = (uint32_t)(i - row * width);
  const uint64_t seed = (uint64_t)seeds[row];
  const uint64_t pos = pos64 ? (uint64_t) reinterpret_cast<const int64_t*>(positions)[row]
                             : (uint64_t)(int64_t) reinterpret_cast<const int32_t*>(positions)[row];
  uint32_t h = 0u;
  h = murmur_block(h, (uint32_t)seed);
  h = murmur_block(h, (uint32_t)(seed >> 32));
  h = murmur_block(h, (uint32_t)pos);
  h = murmur_block(h, col + ((uint32_t)stream_id << 16));
  h = fmix32(h ^ 16u);
  out[i] = (float)(h >> 8) * 5.9604644775390625e-08f;  // 2^-24
}

}  // namespace dsv

using namespace dsv;

extern "C" const char* dsv_last_error(void) { return g_error; }

extern "C" int dsv_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

extern "C" int dsv_uniforms(const int64_t* seeds, const void* positions, int32_t positions_i64, int64_t n,
                            int32_t width, int32_t stream_id, float* out, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (n < 0 || width <= 0 || width >= 65536 || stream_id < 0 || stream_id > 3)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_uniforms: invalid layout (n %lld, width %d, stream %d)", (long long)n, width,
             stream_id);
  if (n == 0) return DSV_OK;
  if (!seeds || !positions || !out) DSV_FAIL(DSV_ERR_INVALID, "dsv_uniforms: null pointer");
  const int64_t total = n * width;
  const int threads = 256;
  hipLaunchKernelGGL(k_uniforms, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, stream,
                     seeds, positions, positions_i64, n, width, stream_id, out);
  DSV_CHECK_LAUNCH("k_uniforms");
  return DSV_OK;
}
