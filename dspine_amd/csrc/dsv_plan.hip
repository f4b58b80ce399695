// SPS verify-length planner for gfx950 (verification/sps.py:35-99): the calibration lookup of
// each draft position's confidence, prefix survival, the global selection of the budget's
// highest-survival positions, per-request verify lengths, the ragged layout's row pointer and
// the compact window index -- one workgroup, one launch, no host synchronisation, so the plan
// can sit inside a captured HIP graph.
//
// Selection order: survival descending, then position-major index (d * bs + b) ascending, the
// order of a stable descending argsort of the transposed survival matrix.  The M = budget - bs
// selected positions are found by a radix select (four 8-bit digit passes of LDS histograms
// over order-preserving 32-bit keys) and a block scan that ranks the ties at the M-th key.
#include <string.h>

#include "dsv_common.h"

namespace dsv {

constexpr int PLAN_THREADS = 1024;
constexpr int PLAN_NW = PLAN_THREADS / WAVE;
constexpr int64_t PLAN_LDS_MAX = 152 * 1024;  // dynamic LDS: keys [bs * gamma] + lengths [bs]

// First index of a sorted float64 array whose value is >= x (torch.bucketize, right=False,
// comparing in float64 as torch does for a float32 input against float64 boundaries).
__device__ __forceinline__ int lower_bound_f64(const double* b, int n, double x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (b[mid] < x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// The bin of confidence x: bucketize against the boundaries, else trunc(x * bins) clamped into
// [0, bins - 1] (a float32 product, as (raw * n_bins).to(int64) computes it; non-finite
// products take bin 0, as the CPU conversion of an out-of-range float gives INT64_MIN).
__device__ __forceinline__ int conf_bin(float x, int n_bins, const double* bounds, int nb) {
  if (bounds) return lower_bound_f64(bounds, nb, (double)x);
  const float y = x * (float)n_bins;
  if (!(y > -1.f)) return 0;  // NaN, -inf and negatives below -1 (their truncation is <= -1)
  if (y >= 9.2233720368547758e18f) return 0;
  const int64_t t = (int64_t)y;
  return t < 0 ? 0 : (t > n_bins - 1 ? n_bins - 1 : (int)t);
}

// Which of a block's 256 digit counts holds the `rem`-th largest element (1-based), counting
// from digit 255 down: returns the digit and leaves the count of larger digits in *above.
// Wave 0 only: lane l sums digits 255 - 4l .. 252 - 4l, a scan over lanes finds the group.
__device__ __forceinline__ int find_digit(const uint32_t* hist, uint32_t rem, uint32_t* above) {
  const int lane = threadIdx.x & (WAVE - 1);
  uint32_t h[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = hist[255 - 4 * lane - j];
    s += h[j];
  }
  const uint32_t incl = wave_incl_scan(s);
  const uint64_t hit = __ballot(incl >= rem);
  const int g = __ffsll((long long)hit) - 1;  // the first group reaching rem (rem <= total)
  const uint32_t before = __builtin_amdgcn_readlane(incl - s, g);
  uint32_t hg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) hg[j] = __builtin_amdgcn_readlane(h[j], g);
  uint32_t cum = before;
  int d = 255 - 4 * g;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (cum + hg[j] >= rem) {
      d = 255 - 4 * g - j;
      break;
    }
    cum += hg[j];
  }
  *above = cum;
  return d;
}

__global__ __launch_bounds__(PLAN_THREADS) void k_sps_plan(const float* raw, int64_t raw_stride, int bs, int gamma,
                                                           const float* prob, int64_t prob_stride, int n_bins,
                                                           int64_t prob_rows, const int64_t* depth,
                                                           const double* bounds, int nb, int budget,
                                                           int32_t* lens_io, int32_t* qo_out, int64_t* index_out) {
  extern __shared__ uint32_t lds[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_rem;
  __shared__ int32_t sred[PLAN_NW];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int full = gamma + 1;
  const int64_t N = (int64_t)bs * gamma;
  uint32_t* key = lds;                                       // [N] survival keys, position-major
  int32_t* lens = reinterpret_cast<int32_t*>(lds + (raw ? N : 0));  // [bs]

  if (raw) {
    // calibration lookup, prefix survival (running product in float64, each prefix rounded to
    // float32, then the running minimum) -- one request a thread
    for (int b = tid; b < bs; b += PLAN_THREADS) {
      const float* r = raw + (int64_t)b * raw_stride;
      double acc = 1.0;
      float run = 0.f;
      for (int d = 0; d < gamma; ++d) {
        int64_t row = depth[d];
        row = row < 0 ? 0 : (row >= prob_rows ? prob_rows - 1 : row);  // (indices must be valid)
        const float c = prob[row * prob_stride + conf_bin(r[d], n_bins, bounds, nb)];
        acc *= (double)c;
        const float s = (float)acc;
        run = d == 0 ? s : fminf(run, s);
        key[(int64_t)d * bs + b] = f32_key(run);
      }
      lens[b] = 1;
    }
    __syncthreads();
    // the M-th largest key (M = budget - bs, 0 <= M <= N) and how many of its ties are taken
    const int64_t M = (int64_t)budget - bs;
    uint32_t kth = 0xFFFFFFFFu, need = 0;
    bool all = M >= N, none = M <= 0;
    if (!all && !none) {
      if (tid == 0) {
        s_prefix = 0;
        s_rem = (uint32_t)M;
      }
      uint32_t mask = 0;
      for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        for (int64_t i = tid; i < N; i += PLAN_THREADS) {
          const uint32_t k = key[i];
          if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < WAVE) {
          uint32_t above = 0;
          const int dg = find_digit(hist, s_rem, &above);
          if (lane == 0) {
            s_prefix = prefix | ((uint32_t)dg << shift);
            s_rem -= above;
          }
        }
        mask |= 0xFFu << shift;
        __syncthreads();
      }
      kth = s_prefix;
      need = s_rem;
    }
    // ties at the M-th key are taken in index order: each thread owns a contiguous index range
    const int64_t per = (N + PLAN_THREADS - 1) / PLAN_THREADS;
    const int64_t i0 = (int64_t)tid * per, i1 = i0 + per < N ? i0 + per : N;
    int my_ties = 0;
    if (!all && !none)
      for (int64_t i = i0; i < i1; ++i) my_ties += key[i] == kth;
    int tot = 0;
    int rank = block_excl_scan<PLAN_NW>(my_ties, sred, &tot);
    for (int64_t i = i0; i < i1; ++i) {
      const uint32_t k = key[i];
      bool take = all;
      if (!all && !none) {
        take = k > kth;
        if (k == kth) take = (uint32_t)(rank++) < need;
      }
      if (take) atomicAdd(&lens[(int)(i % bs)], 1);
    }
    __syncthreads();
  } else {
    // given lengths: only the layout
    for (int b = tid; b < bs; b += PLAN_THREADS) lens[b] = lens_io[b];
    __syncthreads();
  }
  // row pointer (exclusive prefix of the lengths) and the window index, contiguous requests a
  // thread
  const int perb = (bs + PLAN_THREADS - 1) / PLAN_THREADS;
  const int b0 = tid * perb, b1 = b0 + perb < bs ? b0 + perb : bs;
  int mine = 0;
  for (int b = b0; b < b1; ++b) mine += lens[b];
  int total = 0;
  int start = block_excl_scan<PLAN_NW>(mine, sred, &total);
  for (int b = b0; b < b1; ++b) {
    const int n = lens[b];
    if (raw) lens_io[b] = n;
    if (qo_out) qo_out[b] = start;
    // (given lengths that do not sum to the budget -- a caller's error -- write only the
    // index's `budget` entries; qo_indptr[bs] reports their total)
    if (index_out)
      for (int d = 0; d < n; ++d)
        if ((unsigned)(start + d) < (unsigned)budget) index_out[start + d] = (int64_t)b * full + d;
    start += n;
  }
  if (qo_out && tid == 0) qo_out[bs] = total;
}

}  // namespace dsv

using namespace dsv;

extern "C" int dsv_sps_plan(const float* raw, int64_t raw_stride, int32_t bs, int32_t gamma, const float* probabilities,
                            int64_t prob_stride, int32_t n_bins, int64_t prob_rows, const int64_t* depth,
                            const double* boundaries, int32_t n_boundaries, int32_t budget, int32_t* verify_lens,
                            int32_t* qo_indptr, int64_t* window_index, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (bs < 1 || gamma < 1) DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: empty plan (bs %d, gamma %d)", bs, gamma);
  if (!verify_lens) DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: verify_lens is required");
  const int64_t N = (int64_t)bs * gamma;
  if (raw) {
    if (budget < bs || (int64_t)budget > (int64_t)bs * (gamma + 1))
      DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: SPS budget must include every root and fit the draft block");
    if (raw_stride < gamma || !probabilities || !depth || n_bins < 1 || prob_rows < 1 || prob_stride < n_bins)
      DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: invalid confidence / table layout");
    if (boundaries && (n_boundaries < 0 || n_boundaries > n_bins - 1))
      DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: %d boundaries for %d bins", n_boundaries, n_bins);
  }
  if (!raw && window_index && budget < 0) DSV_FAIL(DSV_ERR_INVALID, "dsv_sps_plan: negative budget %d", budget);
  const int64_t lds = ((raw ? N : 0) + bs) * 4;
  if (lds > PLAN_LDS_MAX)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_sps_plan: bs %d x gamma %d exceeds one workgroup's LDS", bs, gamma);
  (void)hipFuncSetAttribute((const void*)k_sps_plan, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(k_sps_plan, dim3(1), dim3(PLAN_THREADS), (size_t)lds, stream, raw, raw_stride, bs, gamma,
                     probabilities, prob_stride, n_bins, prob_rows, depth, boundaries, boundaries ? n_boundaries : 0,
                     budget, verify_lens, qo_indptr, window_index);
  DSV_CHECK_LAUNCH("k_sps_plan");
  return DSV_OK;
}
