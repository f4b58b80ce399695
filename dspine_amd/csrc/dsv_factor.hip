// Factorized draft q table for gfx950 (sampling/factorized/{kernels,cancellation,weights}.py):
// the table of the serial last-write refinement, out[n, j, c] =
//   head[c] . (y / sqrt(mean(y^2) + eps) * norm),   y = x[n] + a[n] * (W m[n, j]),
// evaluated in float64 from a per-model cache so that no [n, K, H] vector is formed:
//   numerator   = base[n, c] + a * (m[n, j] . TG[cand c])     base = (x * norm) . head[c]
//   d = |y|^2   = first + 2 a (x W) . m + a^2 m^T (W^T W) m   first = |x|^2
//   out         = numerator / sqrt(d / H + eps)
// and, where d cancels (d < 2^-24 of |first| + |2a cross| + |a^2 quad|, or not finite), the
// direct form above for that (n, j).  Launches:
//   k_fx_prep     x = raw[state row] (float64), a, first, base (one workgroup a block row)
//   k_fx_msg      m = sigmoid(query + G[sender] + bias) * V[sender], tg = TG[candidate]
//   k_fx_gemm     x W (split over H) and m Gram on the float64 matrix cores
//                 (v_mfma_f64_16x16x4f64, tiles staged in LDS)
//   k_fx_final    m . tg[c] (16 x 16 on the matrix cores), the cross and quadratic terms, the
//                 cancellation test, out
//   k_fx_direct   the direct form for the (n, j) the test rejected (others return at once)
// The cache (weights.py build_cache) is made by k_fx_widen (rows to float64, scaled) and the same
// GEMM with strided operands.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "dsv_common.h"

namespace dsv {

typedef double d4 __attribute__((ext_vector_type(4)));

constexpr int FX_THREADS = 256;
constexpr int GT = 64;   // GEMM tile (rows and columns of C a workgroup computes)
constexpr int GK = 32;   // k depth a tile stage holds
constexpr int GB = 128;  // the large GEMM tile (grids that fill the part), 16 deep a stage
constexpr int GKB = 16;
constexpr int FX_KMAX = 64;
constexpr int FX_SPLIT_MAX = 16;

__device__ __forceinline__ double ld_any(const void* p, int dt, int64_t i) {
  if (dt == DSV_BF16) return (double)__uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
  return (double)reinterpret_cast<const float*>(p)[i];
}

// Block-wide sum in a fixed order (waves by lane tree, then waves in index order).
__device__ __forceinline__ double fx_block_sum(double v, double* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  __syncthreads();
  if (lane == 0) sh[wid] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < FX_THREADS / WAVE; ++i) s += sh[i];
  return s;
}

// ---------------------------------------------------------------------------------------------
// C[M, N] (one split's part) = A[M, K] . B[K, N], float64.  A(m, k) = A[m * am + k * ak],
// B(k, n) = B[k * bk + n * bn]; split z of gridDim.z takes k in [z * kchunk, (z + 1) * kchunk)
// and writes (accumulate: adds to) C + z * M * N (row-major, ldc = N).  A 64 x 64 tile a
// workgroup; each wave a 32 x 32
// quarter as 2 x 2 blocks of 16 x 16.  MFMA operands (v_mfma_f64_16x16x4f64): lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16] of the 16 x 4 / 4 x 16 step and receives
// D[4v + l / 16][l % 16], v = 0..3.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(FX_THREADS) void k_fx_gemm(const double* __restrict__ A, int64_t am, int64_t ak,
                                                       const double* __restrict__ B, int64_t bk, int64_t bn,
                                                       double* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                       int64_t kchunk, int accumulate) {
  constexpr int PER = (GT * GK) / FX_THREADS;  // elements of each operand a thread stages
  __shared__ double As[GT][GK + 1];
  __shared__ double Bs[GK][GT + 1];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
  const int64_t m0 = (int64_t)blockIdx.y * GT, n0 = (int64_t)blockIdx.x * GT;
  const int64_t k_lo = (int64_t)blockIdx.z * kchunk;
  const int64_t k_hi = k_lo + kchunk < K ? k_lo + kchunk : K;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
  const int li = lane & 15, lg = lane >> 4;
  d4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = d4{0.0, 0.0, 0.0, 0.0};
  // the next stage's operands, loaded into registers while the current stage is multiplied.
  // Thread t stages A rows t / GK + e * (256 / GK) at depth t % GK, and B depths
  // t / GT + e * (256 / GT) at column t % GT: one base address each, fixed strides over e.
  static_assert(FX_THREADS % GK == 0 && FX_THREADS % GT == 0, "staging strides");
  constexpr int ARS = FX_THREADS / GK, BKS = FX_THREADS / GT;
  const int a_r = tid / GK, a_k = tid % GK, b_k = tid / GT, b_n = tid % GT;
  const int64_t gn_b = n0 + b_n;
  const double* a_base = A + (m0 + a_r) * am + (k_lo + a_k) * ak;
  const double* b_base = B + (k_lo + b_k) * bk + gn_b * bn;
  double ra[PER], rb[PER];
  auto fetch = [&](int64_t kofs) {
    const bool ka = k_lo + kofs + a_k < k_hi;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const bool ina = ka && m0 + a_r + e * ARS < M;
      ra[e] = ina ? a_base[e * ARS * am + kofs * ak] : 0.0;
      const bool inb = gn_b < N && k_lo + kofs + b_k + e * BKS < k_hi;
      rb[e] = inb ? b_base[(e * BKS + kofs) * bk] : 0.0;
    }
  };
  if (k_lo < k_hi) fetch(0);
  for (int64_t k0 = k_lo; k0 < k_hi; k0 += GK) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      As[a_r + e * ARS][a_k] = ra[e];
      Bs[b_k + e * BKS][b_n] = rb[e];
    }
    __syncthreads();
    if (k0 + GK < k_hi) fetch(k0 + GK - k_lo);
#pragma unroll
    for (int s = 0; s < GK / 4; ++s) {
      double a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[wm + 16 * i + li][4 * s + lg];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[4 * s + lg][wn + 16 * j + li];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  double* Cz = C + (int64_t)blockIdx.z * M * N;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t gm = m0 + wm + 16 * i + 4 * v + lg, gn = n0 + wn + 16 * j + li;
        if (gm < M && gn < N) Cz[gm * N + gn] = accumulate ? Cz[gm * N + gn] + acc[i][j][v] : acc[i][j][v];
      }
}

// A raw buffer over [base, base + bytes): loads past its end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fx_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ double fx_load8(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  const auto t = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)voff, (int)soff, 0);
  return __builtin_bit_cast(double, t);
}
// bytes spanned by a rows x cols operand with element strides (rs, cs), float64
__host__ __device__ __forceinline__ int64_t fx_extent(int64_t rows, int64_t rs, int64_t cols, int64_t cs) {
  return rows > 0 && cols > 0 ? ((rows - 1) * rs + (cols - 1) * cs + 1) * 8 : 0;
}

// The same product on 128 x 128 tiles: each wave a 64 x 64 quarter (4 x 4 MFMA tiles, sixteen
// accumulators), 16-deep stages -- 16 MFMAs a wave for every 8 fragment reads, and a quarter of
// the 64-tile kernel's operand traffic per flop.  For grids of at least a round of workgroups.
__global__ __launch_bounds__(FX_THREADS, 2) void k_fx_gemm_big(const double* __restrict__ A, int64_t am, int64_t ak,
                                                           const double* __restrict__ B, int64_t bk, int64_t bn,
                                                           double* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                           int64_t kchunk, int accumulate) {
  constexpr int PER = (GB * GKB) / FX_THREADS;  // 8 elements of each operand a thread stages
  static_assert(FX_THREADS % GKB == 0 && FX_THREADS % GB == 0, "staging strides");
  constexpr int ARS = FX_THREADS / GKB, BKS = FX_THREADS / GB;  // 16 rows / 2 depths apart
  __shared__ double As[GB][GKB + 1];
  __shared__ double Bs[GKB][GB + 1];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
  const int64_t m0 = (int64_t)blockIdx.y * GB, n0 = (int64_t)blockIdx.x * GB;
  const int64_t k_lo = (int64_t)blockIdx.z * kchunk;
  const int64_t k_hi = k_lo + kchunk < K ? k_lo + kchunk : K;
  const int wm = (w >> 1) * 64, wn = (w & 1) * 64;
  const int li = lane & 15, lg = lane >> 4;
  d4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = d4{0.0, 0.0, 0.0, 0.0};
  // thread t stages A rows t / 16 + 16 e at depth t % 16, and B depths t / 128 + 2 e at column
  // t % 128 (the next stage loaded into registers while the current one is multiplied)
  // (raw buffers over the operands' extents -- under 2 GB, checked by the launcher: 32-bit lane
  // offsets, the stage's k offset a scalar one, no 64-bit address arithmetic per element)
  const int a_r = tid / GKB, a_k = tid % GKB, b_k = tid / GB, b_n = tid % GB;
  const int64_t gn_b = n0 + b_n;
  const auto rsa = fx_rsrc(A, fx_extent(M, am, K, ak));
  const auto rsb = fx_rsrc(B, fx_extent(K, bk, N, bn));
  const uint32_t a_off = (uint32_t)(((m0 + a_r) * am + (k_lo + a_k) * ak) * 8);
  const uint32_t b_off = (uint32_t)(((k_lo + b_k) * bk + gn_b * bn) * 8);
  const uint32_t a_step = (uint32_t)(ARS * am * 8), b_step = (uint32_t)(BKS * bk * 8);
  double ra[PER], rb[PER];
  auto fetch = [&](int64_t kofs) {
    const bool ka = k_lo + kofs + a_k < k_hi;
    const uint32_t sa = (uint32_t)(kofs * ak * 8), sb = (uint32_t)(kofs * bk * 8);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const bool ina = ka && m0 + a_r + e * ARS < M;
      const double xa = fx_load8(rsa, a_off + (uint32_t)e * a_step, sa);
      ra[e] = ina ? xa : 0.0;
      const bool inb = gn_b < N && k_lo + kofs + b_k + e * BKS < k_hi;
      const double xb = fx_load8(rsb, b_off + (uint32_t)e * b_step, sb);
      rb[e] = inb ? xb : 0.0;
    }
  };
  if (k_lo < k_hi) fetch(0);
  for (int64_t k0 = k_lo; k0 < k_hi; k0 += GKB) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      As[a_r + e * ARS][a_k] = ra[e];
      Bs[b_k + e * BKS][b_n] = rb[e];
    }
    __syncthreads();
    if (k0 + GKB < k_hi) fetch(k0 + GKB - k_lo);
#pragma unroll
    for (int s = 0; s < GKB / 4; ++s) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[wm + 16 * i + li][4 * s + lg];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[4 * s + lg][wn + 16 * j + li];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  double* Cz = C + (int64_t)blockIdx.z * M * N;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t gm = m0 + wm + 16 * i + 4 * v + lg, gn = n0 + wn + 16 * j + li;
        if (gm < M && gn < N) Cz[gm * N + gn] = accumulate ? Cz[gm * N + gn] + acc[i][j][v] : acc[i][j][v];
      }
}

// ---------------------------------------------------------------------------------------------
// Per-round kernels
// ---------------------------------------------------------------------------------------------
struct FxP {
  dsv_factor_args a;
  int split;        // parts of x W (over H)
  double* xw_part;  // [split, n, R]
  double* mg;       // [n K, R]
};

// the state row (of bs * T) block row i refines: kernels.py:19-21
__device__ __forceinline__ int64_t fx_source(const dsv_factor_args& a, int64_t i) {
  return i / (a.T - 1) * a.T + i % (a.T - 1) + 1;
}
__device__ __forceinline__ const void* fx_head_row(const dsv_factor_args& a, int64_t i, int c, int64_t& off) {
  if (a.candidate_head) {
    off = (i * a.K + c) * a.head_stride;
    return a.candidate_head;
  }
  int64_t cid = a.cand[i * a.K + c];
  cid = cid < 0 ? 0 : (cid >= a.vocab ? a.vocab - 1 : cid);
  off = cid * a.head_stride;
  return a.head;
}

template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) FxVec {
  T v[VEC];
};
__device__ __forceinline__ double fx_widen(uint16_t v) { return (double)__uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ double fx_widen(float v) { return (double)v; }

// x, a, first (kernels.py:15-27) and base (weights.py:12-31): one workgroup a block row.  Each
// thread takes VEC consecutive h at a time (one 8- or 16-byte load of the raw row and of each of
// the 16 candidates' head rows in flight together); the 16 dot products of a group of candidates
// are reduced with one barrier pair.  RT / HT are uint16_t (bf16 bits) or float.
template <typename RT, typename HT, int VEC>
__global__ __launch_bounds__(FX_THREADS) void k_fx_prep(FxP P) {
  __shared__ double red[FX_THREADS / WAVE][16];
  const dsv_factor_args& a = P.a;
  const int64_t i = blockIdx.x;
  const int64_t src = fx_source(a, i);
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
  const RT* raw = reinterpret_cast<const RT*>(a.raw) + src * a.raw_stride;
  double* xrow = a.x + i * a.H;
  double first = 0.0;
  for (int c0 = 0; c0 < a.K; c0 += 16) {
    const HT* hrow[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      int64_t off = 0;
      const void* hr = fx_head_row(a, i, c0 + c < a.K ? c0 + c : c0, off);
      hrow[c] = reinterpret_cast<const HT*>(hr) + off;
    }
    double base[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) base[c] = 0.0;
    for (int h = tid * VEC; h < a.H; h += FX_THREADS * VEC) {
      const FxVec<RT, VEC> rv = *reinterpret_cast<const FxVec<RT, VEC>*>(raw + h);
      FxVec<HT, VEC> hv[16];
#pragma unroll
      for (int c = 0; c < 16; ++c)
        if (c0 + c < a.K) hv[c] = *reinterpret_cast<const FxVec<HT, VEC>*>(hrow[c] + h);
      double xn[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const double xv = fx_widen(rv.v[e]);
        if (c0 == 0) first += xv * xv;
        xn[e] = xv * a.norm[h + e];
        if (c0 == 0) xrow[h + e] = xv;
      }
#pragma unroll
      for (int c = 0; c < 16; ++c)
        if (c0 + c < a.K) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) base[c] += xn[e] * fx_widen(hv[c].v[e]);
        }
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const double s = wave_sum(base[c]);
      if (lane == 0) red[w][c] = s;
    }
    __syncthreads();
    if (tid < 16 && c0 + tid < a.K) {
      double s = 0.0;
#pragma unroll
      for (int q = 0; q < FX_THREADS / WAVE; ++q) s += red[q][tid];
      a.base_out[i * a.K + c0 + tid] = s;
    }
    __syncthreads();
  }
  first = fx_block_sum(first, &red[0][0]);
  if (tid == 0) {
    a.first[i] = first;
    a.scale[i] = (double)a.rms[src];
  }
}

// the prep instance for the operand dtypes: 8 or 4 elements a load when every row start and
// stride allows it, one element a load otherwise
static void fx_launch_prep(const FxP& P, hipStream_t stream) {
  const dsv_factor_args& a = P.a;
  const void* heads = a.candidate_head ? a.candidate_head : a.head;
  const int vec = (a.raw_dtype == DSV_BF16 && a.head_dtype == DSV_BF16) ? 8 : 4;
  const int rsz = a.raw_dtype == DSV_BF16 ? 2 : 4, hsz = a.head_dtype == DSV_BF16 ? 2 : 4;
  const bool aligned = a.H % vec == 0 && a.raw_stride % vec == 0 && a.head_stride % vec == 0 &&
                       (uintptr_t)a.raw % (rsz * vec) == 0 && (uintptr_t)heads % (hsz * vec) == 0;
  const dim3 grid((unsigned)a.n), block(FX_THREADS);
  const bool rb = a.raw_dtype == DSV_BF16, hb = a.head_dtype == DSV_BF16;
  if (aligned && vec == 8) {
    hipLaunchKernelGGL((k_fx_prep<uint16_t, uint16_t, 8>), grid, block, 0, stream, P);
  } else if (aligned) {
    if (rb) hipLaunchKernelGGL((k_fx_prep<uint16_t, float, 4>), grid, block, 0, stream, P);
    else if (hb) hipLaunchKernelGGL((k_fx_prep<float, uint16_t, 4>), grid, block, 0, stream, P);
    else hipLaunchKernelGGL((k_fx_prep<float, float, 4>), grid, block, 0, stream, P);
  } else if (rb && hb) {
    hipLaunchKernelGGL((k_fx_prep<uint16_t, uint16_t, 1>), grid, block, 0, stream, P);
  } else if (rb) {
    hipLaunchKernelGGL((k_fx_prep<uint16_t, float, 1>), grid, block, 0, stream, P);
  } else if (hb) {
    hipLaunchKernelGGL((k_fx_prep<float, uint16_t, 1>), grid, block, 0, stream, P);
  } else {
    hipLaunchKernelGGL((k_fx_prep<float, float, 1>), grid, block, 0, stream, P);
  }
}

// m and tg of every (i, j) (kernels.py:30-67): one workgroup a block row
__global__ __launch_bounds__(FX_THREADS) void k_fx_msg(FxP P) {
  const dsv_factor_args& a = P.a;
  const int64_t i = blockIdx.x;
  const int64_t req = i / (a.T - 1), pos = i % (a.T - 1);
  const int64_t src = req * a.T + pos + 1;
  // four elements a thread at a time: their operands loaded together, then computed and stored
  constexpr int U = 4;
  const int total = a.K * a.R;
  for (int idx0 = threadIdx.x; idx0 < total; idx0 += FX_THREADS * U) {
    double q[U], g[U], bs[U], vm[U], tgv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = idx0 + u * FX_THREADS;
      const int id = idx < total ? idx : total - 1;
      const int j = id / a.R, r = id % a.R;
      int64_t sid = pos == 0 ? a.anchors[req] : a.cand[(i - 1) * a.K + j];
      int64_t cid = a.cand[i * a.K + j];
      sid = sid < 0 ? 0 : (sid >= a.vocab ? a.vocab - 1 : sid);
      cid = cid < 0 ? 0 : (cid >= a.vocab ? a.vocab - 1 : cid);
      q[u] = ld_any(a.query, a.query_dtype, src * a.query_stride + r);
      g[u] = a.G[sid * a.R + r];
      bs[u] = a.bias[r];
      vm[u] = a.Vm[sid * a.R + r];
      tgv[u] = a.TG[cid * a.R + r];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = idx0 + u * FX_THREADS;
      if (idx >= total) continue;
      const double gate = q[u] + g[u] + bs[u];
      const double sig = 1.0 / (1.0 + exp(-gate));
      a.message[i * total + idx] = sig * vm[u];
      a.tg[i * total + idx] = tgv[u];
    }
  }
}

// The finalize (kernels.py:70-123): product m . tg on the matrix cores, cross and quadratic on
// the vector units, the cancellation test, out.  One workgroup a block row (K <= 16 on the matrix
// path; wider K on the vector units).
__global__ __launch_bounds__(FX_THREADS) void k_fx_final(FxP P) {
  __shared__ double xw[1024];
  __shared__ double prod[16 * 16 * (FX_THREADS / WAVE)];
  __shared__ double den_s[FX_KMAX];
  const dsv_factor_args& a = P.a;
  const int64_t i = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
  const int K = a.K, R = a.R;
  // x W for this row: the split parts summed in order (eight parts' loads in flight together)
  for (int r = tid; r < R; r += FX_THREADS) {
    double s = 0.0;
    int z = 0;
    for (; z + 8 <= P.split; z += 8) {
      double pz[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) pz[u] = P.xw_part[((int64_t)(z + u) * a.n + i) * R + r];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += pz[u];
    }
    for (; z < P.split; ++z) s += P.xw_part[((int64_t)z * a.n + i) * R + r];
    xw[r] = s;
  }
  const double* msg = a.message + i * K * R;
  const double* tgr = a.tg + i * K * R;
  // product[j][c] = m_j . tg_c: 16 x 16 from R in steps of 4, the R range split over the waves
  if (K <= 16) {
    const int li = lane & 15, lg = lane >> 4;
    d4 acc = {0.0, 0.0, 0.0, 0.0};
    const int per = (R + 4 * (FX_THREADS / WAVE) - 1) / (4 * (FX_THREADS / WAVE)) * 4;
    const int r_lo = w * per, r_hi = r_lo + per < R ? r_lo + per : R;
    // eight 4-deep steps' operands loaded together, then their products in step order
    for (int r0 = r_lo; r0 < r_hi; r0 += 32) {
      double av[8], bv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = r0 + 4 * u + lg;
        const bool in = li < K && r < r_hi;
        av[u] = in ? msg[(int64_t)li * R + r] : 0.0;
        bv[u] = in ? tgr[(int64_t)li * R + r] : 0.0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (r0 + 4 * u < r_hi) acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[u], bv[u], acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) prod[w * 256 + (4 * v + lg) * 16 + li] = acc[v];
  }
  __syncthreads();
  // cross_j = xw . m_j and quad_j = mg_j . m_j: 16 lanes a j (K <= 16), the R range split
  const int grp = tid / 16, gl = tid % 16;
  for (int j0 = 0; j0 < K; j0 += FX_THREADS / 16) {
    const int j = j0 + grp;
    double cr = 0.0, qd = 0.0;
    if (j < K) {
      const double* mj = msg + (int64_t)j * R;
      const double* gj = P.mg + (i * K + j) * R;
      // eight steps' loads in flight together, summed in step order
      for (int r0 = gl; r0 < R; r0 += 128) {
        double mv[8], gv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int r = r0 + 16 * u;
          mv[u] = r < R ? mj[r] : 0.0;
          gv[u] = r < R ? gj[r] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (r0 + 16 * u < R) {
            cr += xw[r0 + 16 * u] * mv[u];
            qd += gv[u] * mv[u];
          }
      }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
      cr += __shfl_xor(cr, o, 16);
      qd += __shfl_xor(qd, o, 16);
    }
    if (j < K && gl == 0) {
      const double sc = a.scale[i], first = a.first[i];
      const double second = 2.0 * sc * cr;
      const double third = sc * sc * qd;
      const double d = first + second + third;
      const double mag = fabs(first) + fabs(second) + fabs(third);
      const bool safe = isfinite(d) && isfinite(mag) && d >= 0.0 && (mag == 0.0 || d > 0x1p-24 * mag);
      a.safe[i * K + j] = safe ? 1 : 0;
      a.d[i * K + j] = d;
      a.magnitude[i * K + j] = mag;
      den_s[j] = sqrt(d / (double)a.H + a.eps);
    }
  }
  __syncthreads();
  for (int idx = tid; idx < K * K; idx += FX_THREADS) {
    const int j = idx / K, c = idx % K;
    double pr;
    if (K <= 16) {
      pr = 0.0;
      for (int q = 0; q < FX_THREADS / WAVE; ++q) pr += prod[q * 256 + j * 16 + c];
    } else {
      pr = 0.0;
      for (int r = 0; r < R; ++r) pr += msg[(int64_t)j * R + r] * tgr[(int64_t)c * R + r];
    }
    const double num = a.base_out[i * K + c] + a.scale[i] * pr;
    a.out[(i * K + j) * K + c] = (float)(num / den_s[j]);
  }
}

// The direct form (cancellation.py:16-79) for the (i, j) the test rejected; one workgroup each.
__global__ __launch_bounds__(FX_THREADS) void k_fx_direct(FxP P) {
  __shared__ double red[FX_THREADS / WAVE];
  __shared__ double m[1024];
  const dsv_factor_args& a = P.a;
  const int64_t ij = blockIdx.x;
  if (a.safe[ij]) return;
  const int64_t i = ij / a.K;
  const int K = a.K, R = a.R, H = a.H;
  for (int r = threadIdx.x; r < R; r += FX_THREADS) m[r] = a.message[ij * R + r];
  __syncthreads();
  const double sc = a.scale[i];
  double sq = 0.0;
  double* y = a.y + ij * H;
  for (int h = threadIdx.x; h < H; h += FX_THREADS) {
    double delta = 0.0;
    const double* wr = a.W + (int64_t)h * R;
    for (int r = 0; r < R; ++r) delta += wr[r] * m[r];
    const double yv = a.x[i * H + h] + sc * delta;
    y[h] = yv;
    sq += yv * yv;
  }
  sq = fx_block_sum(sq, red);
  const double den = sqrt(sq / (double)H + a.eps);
  for (int c = 0; c < K; ++c) {
    int64_t off;
    const void* hr = fx_head_row(a, i, c, off);
    double v = 0.0;
    for (int h = threadIdx.x; h < H; h += FX_THREADS) v += y[h] / den * a.norm[h] * ld_any(hr, a.head_dtype, off + h);
    v = fx_block_sum(v, red);
    if (threadIdx.x == 0) a.out[ij * K + c] = (float)v;
  }
}

// ---------------------------------------------------------------------------------------------
// Cache rows (weights.py:34-80): out[r, :] = scale * widen(src[r, :]) (* mul[:] when given)
// ---------------------------------------------------------------------------------------------
__global__ void k_fx_widen(const void* src, int dt, int64_t stride, int64_t rows, int64_t cols, double scale,
                           const double* mul, double* out) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    double v = scale * ld_any(src, dt, r * stride + c);
    if (mul) v = v * mul[c];
    out[e] = v;
  }
}

}  // namespace dsv

using namespace dsv;

// the most parts x W's depth H is cut into (parts of >= 256)
static int fx_split_cap(int32_t H) {
  int s = 1;
  while (s < FX_SPLIT_MAX && H / (2 * s) >= 256) s *= 2;
  return s;
}
static int fx_split(int64_t n, int32_t R, int32_t H) {
  // enough workgroups over n x R (128-wide) tiles to fill the part
  const int64_t tiles = ((n + GB - 1) / GB) * ((R + GB - 1) / GB);
  int s = 1;
  while (s < fx_split_cap(H) && tiles * s < 512) s *= 2;
  return s;
}

// (a bound that grows with n: a buffer sized for n serves every smaller n)
extern "C" int64_t dsv_factor_workspace_doubles(int64_t n, int32_t K, int32_t H, int32_t R) {
  return (int64_t)fx_split_cap(H) * n * R + n * (int64_t)K * R;
}

static void fx_gemm(const double* A, int64_t am, int64_t ak, const double* B, int64_t bk, int64_t bn, double* C,
                    int64_t M, int64_t N, int64_t K, int split, int accumulate, hipStream_t stream) {
  const int64_t big_tiles = ((N + GB - 1) / GB) * ((M + GB - 1) / GB) * split;
  // (a round of 128-tile workgroups, two a CU; operands addressed by 32-bit buffer offsets)
  const bool big = big_tiles >= 240 && fx_extent(M, am, K, ak) < (1ll << 31) && fx_extent(K, bk, N, bn) < (1ll << 31);
  const int gk = big ? GKB : GK;
  int64_t kchunk = (K + split - 1) / split;
  kchunk = (kchunk + gk - 1) / gk * gk;
  if (big) {
    const dim3 grid((unsigned)((N + GB - 1) / GB), (unsigned)((M + GB - 1) / GB), (unsigned)split);
    hipLaunchKernelGGL(k_fx_gemm_big, grid, dim3(FX_THREADS), 0, stream, A, am, ak, B, bk, bn, C, M, N, K, kchunk,
                       accumulate);
  } else {
    const dim3 grid((unsigned)((N + GT - 1) / GT), (unsigned)((M + GT - 1) / GT), (unsigned)split);
    hipLaunchKernelGGL(k_fx_gemm, grid, dim3(FX_THREADS), 0, stream, A, am, ak, B, bk, bn, C, M, N, K, kchunk,
                       accumulate);
  }
}

static int fx_check_layout(const dsv_factor_args* args, const char* what) {
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "%s: null arguments", what);
  const dsv_factor_args& a = *args;
  if (a.n < 0 || a.K < 1 || a.K > FX_KMAX || a.T < 2 || a.n % (a.T - 1) || a.H < 1 || a.R < 1 || a.vocab < 1)
    DSV_FAIL(DSV_ERR_INVALID, "%s: layout mismatch (n %lld, K %d, T %d, H %d, R %d)", what, (long long)a.n, a.K, a.T,
             a.H, a.R);
  if (a.R > 1024) DSV_FAIL(DSV_ERR_UNSUPPORTED, "%s: rank R %d above 1024", what, a.R);
  if (a.head_dtype != DSV_BF16 && a.head_dtype != DSV_F32)
    DSV_FAIL(DSV_ERR_INVALID, "%s: the head must be bf16 or float32", what);
  if ((!a.head && !a.candidate_head) || a.head_stride < a.H || !a.cand || !a.W || !a.norm || !a.out || !a.x ||
      !a.scale || !a.message || !a.safe || !a.y)
    DSV_FAIL(DSV_ERR_INVALID, "%s: required pointer is null", what);
  return DSV_OK;
}

// The direct form alone (cancellation.py:82-147 apply_direct_fallback) for the (n, j) whose
// safe flag is 0, from x, a, m and the cache's W / norm / head.
extern "C" int dsv_factor_direct(const dsv_factor_args* args, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int rc = fx_check_layout(args, "dsv_factor_direct");
  if (rc != DSV_OK) return rc;
  if (args->n == 0) return DSV_OK;
  FxP P;
  memset(&P, 0, sizeof(P));
  P.a = *args;
  hipLaunchKernelGGL(k_fx_direct, dim3((unsigned)(args->n * args->K)), dim3(FX_THREADS), 0, stream, P);
  DSV_CHECK_LAUNCH("k_fx_direct");
  return DSV_OK;
}

extern "C" int dsv_factor_table(const dsv_factor_args* args, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int rc = fx_check_layout(args, "dsv_factor_table");
  if (rc != DSV_OK) return rc;
  const dsv_factor_args& a = *args;
  if (a.n == 0) return DSV_OK;
  for (int dt : {a.raw_dtype, a.query_dtype, a.head_dtype})
    if (dt != DSV_BF16 && dt != DSV_F32) DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_table: operands must be bf16 or float32");
  if (!a.raw || !a.rms || !a.query || !a.anchors || !a.cand || !a.W || !a.gram || !a.G || !a.Vm || !a.TG || !a.bias ||
      !a.norm || (!a.head && !a.candidate_head) || !a.out || !a.base_out || !a.x || !a.scale || !a.first ||
      !a.message || !a.tg || !a.safe || !a.d || !a.magnitude || !a.y || !a.gemm_ws)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_table: required pointer is null");
  if (a.raw_stride < a.H || a.query_stride < a.R || a.head_stride < a.H)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_table: row strides below the row widths");
  if (a.gemm_ws_doubles < dsv_factor_workspace_doubles(a.n, a.K, a.H, a.R))
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_factor_table: GEMM workspace too small");
  FxP P;
  memset(&P, 0, sizeof(P));
  P.a = a;
  P.split = fx_split(a.n, a.R, a.H);
  P.xw_part = a.gemm_ws;
  P.mg = a.gemm_ws + (int64_t)P.split * a.n * a.R;
  const unsigned n = (unsigned)a.n;
  fx_launch_prep(P, stream);
  hipLaunchKernelGGL(k_fx_msg, dim3(n), dim3(FX_THREADS), 0, stream, P);
  DSV_CHECK_LAUNCH("k_fx_prep / k_fx_msg");
  // x W [n, R] (split over H) and m Gram [n K, R]
  fx_gemm(a.x, a.H, 1, a.W, a.R, 1, P.xw_part, a.n, a.R, a.H, P.split, 0, stream);
  fx_gemm(a.message, a.R, 1, a.gram, a.R, 1, P.mg, a.n * a.K, a.R, a.R, 1, 0, stream);
  DSV_CHECK_LAUNCH("k_fx_gemm");
  hipLaunchKernelGGL(k_fx_final, dim3(n), dim3(FX_THREADS), 0, stream, P);
  hipLaunchKernelGGL(k_fx_direct, dim3((unsigned)(a.n * a.K)), dim3(FX_THREADS), 0, stream, P);
  DSV_CHECK_LAUNCH("k_fx_final / k_fx_direct");
  return DSV_OK;
}

extern "C" int dsv_factor_widen(const void* src, int32_t dtype, int64_t stride, int64_t rows, int64_t cols,
                                double scale, const double* mul, double* out, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!src || !out || rows < 0 || cols < 0 || stride < cols || (dtype != DSV_BF16 && dtype != DSV_F32))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_widen: invalid operands");
  if (rows == 0 || cols == 0) return DSV_OK;
  const int64_t total = rows * cols;
  const unsigned grid = (unsigned)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  hipLaunchKernelGGL(k_fx_widen, dim3(grid), dim3(256), 0, stream, src, dtype, stride, rows, cols, scale, mul, out);
  DSV_CHECK_LAUNCH("k_fx_widen");
  return DSV_OK;
}

extern "C" int dsv_factor_gemm(const double* A, int64_t am, int64_t ak, const double* B, int64_t bk, int64_t bn,
                               double* C, int64_t M, int64_t N, int64_t K, int32_t accumulate, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!A || !B || !C || M < 0 || N < 0 || K < 0) DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_gemm: invalid operands");
  if (M == 0 || N == 0) return DSV_OK;
  if (K == 0) DSV_FAIL(DSV_ERR_INVALID, "dsv_factor_gemm: empty inner dimension");
  fx_gemm(A, am, ak, B, bk, bn, C, M, N, K, 1, accumulate ? 1 : 0, stream);
  DSV_CHECK_LAUNCH("k_fx_gemm");
  return DSV_OK;
}
