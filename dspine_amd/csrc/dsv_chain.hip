// Explicit-distribution entry points for gfx950: in-place logit adjustments, padding rows,
// the compact window index, p > 0 compression, chain rejection on given target / draft
// distributions (dense or packed P, dense or sparse q), and the draft-side K-lane chain.
//
// Semantics follow sampling/compact.py:14-79, sampling/padding.py:4-12,
// verification/sps.py:27-32, sampling/sparse/accept.py:7-78,81-543, sampling/rejection.py:12-153
// and kernels/dspine.py:616-772.
#include <string.h>

#include <type_traits>

#include "dsv_device.h"

namespace dsv {

// ---------------------------------------------------------------------------------------
// Logit adjustments (sampling/compact.py:14-79), in place, one pass per operation, each
// rounded to the logits dtype as the reference's in-place tensor ops are.
// ---------------------------------------------------------------------------------------
constexpr int ADJ_THREADS = 256;

template <typename E>
__device__ __forceinline__ float elem_load(const E* p);
template <>
__device__ __forceinline__ float elem_load<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float elem_load<uint16_t>(const uint16_t* p) {
  return bf16_bits_to_f32(*p);
}
__device__ __forceinline__ void elem_store(float* p, float x) { *p = x; }
__device__ __forceinline__ void elem_store(uint16_t* p, float x) { *p = (uint16_t)f32_to_bf16_bits(x); }

__device__ __forceinline__ int64_t request_of_row(const int64_t* row_to_request, int32_t rows_per_request, int64_t r) {
  return row_to_request ? row_to_request[r] : r / rows_per_request;
}

__device__ __forceinline__ float adjust_one(float x, float s, int32_t op) {
  return op == DSV_ADJ_ADD ? x + s : (x < 0.f ? x * s : x / s);
}

// One element a thread a step (any alignment).
template <typename E>
__global__ __launch_bounds__(ADJ_THREADS) void k_adjust(E* logits, int64_t vocab, int64_t row_stride,
                                                       const int64_t* row_to_request, int32_t rows_per_request,
                                                       int32_t op, const float* values, int64_t values_stride) {
  const int64_t r = blockIdx.y;
  const int64_t req = request_of_row(row_to_request, rows_per_request, r);
  E* row = logits + r * row_stride;
  const float* v = values + req * values_stride;
  for (int64_t j = (int64_t)blockIdx.x * ADJ_THREADS + threadIdx.x; j < vocab; j += (int64_t)gridDim.x * ADJ_THREADS)
    elem_store(row + j, adjust_one(elem_load<E>(row + j), v[j], op));
}

// Eight consecutive elements a thread a step, 16-byte loads and stores (rows and value rows
// 16-byte aligned); the row's last vocab % 8 elements one at a time.
constexpr int ADJ_VEC = 8;
// Eight bf16 values (one 16-byte vector) adjusted with their eight operands.
template <typename E, int OP>
__device__ __forceinline__ void adjust_vec8(uint4& w, const float (&s)[8]) {
  if constexpr (sizeof(E) == 2) {
    uint32_t* wp = reinterpret_cast<uint32_t*>(&w);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = adjust_one(bf16_bits_to_f32(wp[k] & 0xFFFFu), s[2 * k], OP);
      const float hi = adjust_one(bf16_bits_to_f32(wp[k] >> 16), s[2 * k + 1], OP);
      wp[k] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
  }
}
// Up to ADJ_ROWS consecutive rows a workgroup: their logits vectors go out together, and a
// request's eight operands are read again only when the next row belongs to another request
// (compact rows of one request are consecutive).
constexpr int ADJ_ROWS = 4;
template <typename E, int OP>
__global__ __launch_bounds__(ADJ_THREADS) void k_adjust_vec(E* logits, int64_t vocab, int64_t row_stride,
                                                           int64_t rows, const int64_t* row_to_request,
                                                           int32_t rows_per_request, const float* values,
                                                           int64_t values_stride) {
  constexpr int NV = sizeof(E) == 2 ? 1 : 2;  // 16-byte vectors a row holds of eight values
  const int64_t ra = (int64_t)blockIdx.y * ADJ_ROWS;
  int64_t req[ADJ_ROWS];
#pragma unroll
  for (int t = 0; t < ADJ_ROWS; ++t) req[t] = ra + t < rows ? request_of_row(row_to_request, rows_per_request, ra + t) : -1;
  const int64_t step = (int64_t)gridDim.x * ADJ_THREADS * ADJ_VEC;
  for (int64_t j = ((int64_t)blockIdx.x * ADJ_THREADS + threadIdx.x) * ADJ_VEC; j < vocab; j += step) {
    if (j + ADJ_VEC <= vocab) {
      uint4 w[ADJ_ROWS][NV];
#pragma unroll
      for (int t = 0; t < ADJ_ROWS; ++t)
        if (req[t] >= 0)
#pragma unroll
          for (int h = 0; h < NV; ++h)
            w[t][h] = *reinterpret_cast<const uint4*>(logits + (ra + t) * row_stride + j + h * (16 / sizeof(E)));
      float s[8];
      int64_t cur = -1;
#pragma unroll
      for (int t = 0; t < ADJ_ROWS; ++t) {
        if (req[t] < 0) continue;
        if (req[t] != cur) {
          const float* v = values + req[t] * values_stride + j;
          const float4 s0 = *reinterpret_cast<const float4*>(v), s1 = *reinterpret_cast<const float4*>(v + 4);
          s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w;
          s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;
          cur = req[t];
        }
        if constexpr (sizeof(E) == 2) {
          adjust_vec8<E, OP>(w[t][0], s);
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float* x = reinterpret_cast<float*>(&w[t][h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = adjust_one(x[e], s[4 * h + e], OP);
          }
        }
#pragma unroll
        for (int h = 0; h < NV; ++h)
          *reinterpret_cast<uint4*>(logits + (ra + t) * row_stride + j + h * (16 / sizeof(E))) = w[t][h];
      }
    } else {
#pragma unroll
      for (int t = 0; t < ADJ_ROWS; ++t) {
        if (req[t] < 0) continue;
        E* row = logits + (ra + t) * row_stride;
        const float* v = values + req[t] * values_stride;
        for (int64_t k = j; k < vocab; ++k) elem_store(row + k, adjust_one(elem_load<E>(row + k), v[k], OP));
      }
    }
  }
}

// The contiguous layout (rows_per_request rows a request, no row map): a thread's eight values
// are read once and applied to each of the request's rows, ADJ_ROWS rows' loads in flight at a
// time -- a request's value row crosses HBM once instead of once per row.
template <typename E, int OP>
__global__ __launch_bounds__(ADJ_THREADS) void k_adjust_req(E* logits, int64_t vocab, int64_t row_stride,
                                                           int64_t rows, int32_t rows_per_request,
                                                           const float* values, int64_t values_stride) {
  static_assert(sizeof(E) == 2, "bf16 rows");
  const int64_t req = blockIdx.y;
  const int64_t r0 = req * rows_per_request;
  const int64_t r1 = r0 + rows_per_request < rows ? r0 + rows_per_request : rows;
  const float* v = values + req * values_stride;
  const int64_t step = (int64_t)gridDim.x * ADJ_THREADS * ADJ_VEC;
  for (int64_t j = ((int64_t)blockIdx.x * ADJ_THREADS + threadIdx.x) * ADJ_VEC; j < vocab; j += step) {
    if (j + ADJ_VEC <= vocab) {
      const float4 s0 = *reinterpret_cast<const float4*>(v + j), s1 = *reinterpret_cast<const float4*>(v + j + 4);
      const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      for (int64_t rb = r0; rb < r1; rb += ADJ_ROWS) {
        uint4 w[ADJ_ROWS];
#pragma unroll
        for (int t = 0; t < ADJ_ROWS; ++t)
          if (rb + t < r1) w[t] = *reinterpret_cast<const uint4*>(logits + (rb + t) * row_stride + j);
#pragma unroll
        for (int t = 0; t < ADJ_ROWS; ++t) {
          if (rb + t < r1) {
            adjust_vec8<E, OP>(w[t], s);
            *reinterpret_cast<uint4*>(logits + (rb + t) * row_stride + j) = w[t];
          }
        }
      }
    } else {
      for (int64_t r = r0; r < r1; ++r)
        for (int64_t k = j; k < vocab; ++k)
          elem_store(logits + r * row_stride + k, adjust_one(elem_load<E>(logits + r * row_stride + k), v[k], OP));
    }
  }
}

// Presence then repetition on each request's history tokens (each token once), in place.
// One workgroup per row: the history becomes an LDS bitmap, then its set bits are visited.
template <typename E>
__global__ __launch_bounds__(ADJ_THREADS) void k_adjust_history(E* logits, int64_t vocab, int64_t row_stride,
                                                               const int64_t* row_to_request, int32_t rows_per_request,
                                                               const int32_t* hist_ids, int32_t hist_len,
                                                               const float* presence, const float* repetition) {
  extern __shared__ __align__(16) unsigned char dyn[];
  uint32_t* bm = reinterpret_cast<uint32_t*>(dyn);
  const int64_t r = blockIdx.x;
  const int64_t req = request_of_row(row_to_request, rows_per_request, r);
  const int words = (int)((vocab + 31) / 32);
  for (int i = threadIdx.x; i < words; i += ADJ_THREADS) bm[i] = 0u;
  __syncthreads();
  const int32_t* h = hist_ids + req * hist_len;
  for (int i = threadIdx.x; i < hist_len; i += ADJ_THREADS) {
    const int64_t t = h[i];
    if (t >= 0 && t < vocab) atomicOr(&bm[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  const float pres = presence ? presence[req] : 0.f;
  const float rep = repetition ? repetition[req] : 1.f;
  E* row = logits + r * row_stride;
  for (int i = threadIdx.x; i < words; i += ADJ_THREADS) {
    uint32_t w = bm[i];
    while (w) {
      const int e = __ffs(w) - 1;
      w &= w - 1u;
      const int64_t j = (int64_t)i * 32 + e;
      float x = elem_load<E>(row + j);
      if (presence) {
        x -= pres;
        if constexpr (sizeof(E) == 2) x = bf16_bits_to_f32(f32_to_bf16_bits(x));
      }
      if (repetition) x = x < 0.f ? x * rep : x / rep;
      elem_store(row + j, x);
    }
  }
}

// Padding rows (sampling/padding.py:4-12): [0, -inf, -inf, ...].
template <typename E>
__global__ __launch_bounds__(ADJ_THREADS) void k_padding(E* out, int64_t vocab, int64_t row_stride) {
  E* row = out + (int64_t)blockIdx.y * row_stride;
  for (int64_t j = (int64_t)blockIdx.x * ADJ_THREADS + threadIdx.x; j < vocab; j += (int64_t)gridDim.x * ADJ_THREADS)
    elem_store(row + j, j == 0 ? 0.f : -INFINITY);
}

// Compact window index (verification/sps.py:27-32): out[qo[b] + d] = b * T + d, d < qo[b+1]-qo[b].
// Writes stay inside out[0, total) and at most T entries a request.
__global__ void k_window_index(const void* qo, int32_t qo_i64, int32_t T, int64_t* out, int64_t total) {
  const int b = blockIdx.x;
  const int64_t start = load_index(qo, qo_i64, b), end = load_index(qo, qo_i64, b + 1);
  for (int64_t d = threadIdx.x; d < end - start && d < T; d += blockDim.x)
    if (start + d >= 0 && start + d < total) out[start + d] = (int64_t)b * T + d;
}

// ---------------------------------------------------------------------------------------
// compress_probs (sampling/sparse/accept.py:7-78,422-460): per row, the ids with p > 0 in id
// order up to capacity; length = min(n, capacity); overflow = n > capacity or any negative,
// NaN or infinite value; unused slots (-1, 0).  One workgroup per row, tiles of 4096 ids.
// ---------------------------------------------------------------------------------------
constexpr int CMP_THREADS = 512;
constexpr int CMP_E = 8;  // consecutive ids a thread per tile
constexpr int CMP_AHEAD = 4;  // tiles whose loads are in flight

__global__ __launch_bounds__(CMP_THREADS) void k_compress(const float* p, int64_t vocab, int64_t row_stride,
                                                          int32_t capacity, int32_t* ids, float* values,
                                                          int32_t* lengths, int32_t* overflow) {
  constexpr int NW = CMP_THREADS / WAVE;
  constexpr int64_t TILE = (int64_t)CMP_THREADS * CMP_E;
  __shared__ int32_t red[NW];
  __shared__ int32_t s_bad;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const float* row = p + r * row_stride;
  int32_t* oid = ids + r * capacity;
  float* oval = values + r * capacity;
  const bool vec = (uintptr_t)row % 16 == 0;  // (CMP_E ids a thread: 16-byte loads)
  if (tid == 0) s_bad = 0;
  // a tile's CMP_E values of this thread
  auto fetch = [&](int64_t t0, float (&x)[CMP_E]) {
    const int64_t j0 = t0 + (int64_t)tid * CMP_E;
    if (vec && j0 + CMP_E <= vocab) {
#pragma unroll
      for (int h = 0; h < CMP_E / 4; ++h) {
        const float4 u = *reinterpret_cast<const float4*>(row + j0 + 4 * h);
        x[4 * h] = u.x; x[4 * h + 1] = u.y; x[4 * h + 2] = u.z; x[4 * h + 3] = u.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < CMP_E; ++e) x[e] = j0 + e < vocab ? row[j0 + e] : 0.f;
    }
  };
  int64_t total = 0;  // kept ids before the current tile
  bool bad = false;
  // CMP_AHEAD tiles' loads in flight: a ring of registers, the tile loop unrolled by its size so
  // that every slot index is static; a slot is refilled with the tile CMP_AHEAD further on as
  // soon as its values are taken
  float xr[CMP_AHEAD][CMP_E];
#pragma unroll
  for (int d = 0; d < CMP_AHEAD; ++d)
    if ((int64_t)d * TILE < vocab) fetch((int64_t)d * TILE, xr[d]);
  bool done = false;
  for (int64_t tg = 0; tg < vocab && !done; tg += CMP_AHEAD * TILE) {
#pragma unroll
    for (int d = 0; d < CMP_AHEAD; ++d) {
      const int64_t t0 = tg + (int64_t)d * TILE;
      if (done || t0 >= vocab) break;
      float x[CMP_E];
#pragma unroll
      for (int e = 0; e < CMP_E; ++e) x[e] = xr[d][e];
      if (t0 + CMP_AHEAD * TILE < vocab) fetch(t0 + CMP_AHEAD * TILE, xr[d]);
      const int64_t j0 = t0 + (int64_t)tid * CMP_E;
      int32_t cnt = 0;
#pragma unroll
      for (int e = 0; e < CMP_E; ++e) {
        cnt += x[e] > 0.f;
        bad |= x[e] < 0.f || x[e] != x[e] || fabsf(x[e]) == INFINITY;
      }
      int32_t tot = 0;
      int64_t at = total + block_excl_scan<NW>(cnt, red, &tot);
#pragma unroll
      for (int e = 0; e < CMP_E; ++e)
        if (x[e] > 0.f) {
          if (at < capacity) {
            oid[at] = (int32_t)(j0 + e);
            oval[at] = x[e];
          }
          ++at;
        }
      total += tot;
      // more than capacity kept ids: the row overflows whatever the rest holds, and the first
      // capacity ids are written (total is the same in every thread)
      if (total > capacity) done = true;
    }
  }
  if (bad) s_bad = 1;
  __syncthreads();
  for (int64_t i = total + tid; i < capacity; i += CMP_THREADS) {
    oid[i] = -1;
    oval[i] = 0.f;
  }
  if (tid == 0) {
    lengths[r] = (int32_t)(total < capacity ? total : capacity);
    overflow[r] = (total > capacity || s_bad) ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------------------
// Chain rejection on given distributions (sampling/rejection.py:12-98 with dense P and Q;
// sampling/sparse/accept.py:226-419 with dense or packed P and sparse q).  One workgroup per
// request.  Accept draft s iff q > 0, q <= 1 and float32(u*q) < p.  Bonus: the residual
// max(P - q, 0) (P when every draft was accepted or the residual has no mass), inverse CDF in
// id order (float64 sums): the row's tiles give tile masses, the tile holding u*mass is
// scanned, then the thread holding it.  Dense P subtracts the clamped q of the last lane with
// an id; packed P the clamped q summed over the lanes with its id (accept.py:163-166,186-193).
// ---------------------------------------------------------------------------------------
constexpr int CH_THREADS = 1024;                 // (sixteen waves: the loads in flight of one CU)
constexpr int CH_NW = CH_THREADS / WAVE;
constexpr int CH_E = 4;                          // consecutive ids a thread per tile
constexpr int CH_TILE = CH_THREADS * CH_E;       // 4096
constexpr int CH_TILES_MAX = 128;                // vocab <= 524288
constexpr int CH_PACK_MAX = 64;                  // packed capacity handled by one wave

struct ChainShared {
  double red_d[CH_NW];
  int32_t red_i[CH_NW];
  double tile_mass[CH_TILES_MAX];
  double tile_wave[CH_TILES_MAX * CH_NW];  // each wave's part of a tile's mass
  int64_t qid[QMAX];
  float qc[QMAX];       // clamped q of the lane
  int32_t qlast[QMAX];  // last lane with its id
  double qd[QMAX];      // dense P: P - max(P - q, 0) at the lane's id (last lanes), else 0
  int32_t acc;
  int32_t pure;
  int32_t tile, pick_thread;
  double thr, tile_lo, pick_lo;
  double mass;  // the tiles' total (wave scan)
  int64_t bonus;
};

__device__ __forceinline__ int64_t chain_row(const dsv_chain_args& a, int b, int s) {
  const int64_t base = a.row_offsets ? load_index(a.row_offsets, a.row_offsets_i64, b) : (int64_t)b * a.T;
  return base + s;
}

// P of row `row` at id j from its dense storage (RAW: divided by the row's denominator).
__device__ __forceinline__ float chain_dense_p(const dsv_chain_args& a, int64_t row, int64_t j) {
  float p = a.dense_p[row * a.p_stride + j];
  if (a.denominator) p = p / a.denominator[row];
  return p;
}

// Packed rows: those whose overflow flag is 0, and every row when there is no dense fallback
// (where the reference asserts that no row overflowed, its packed prefix is used).
__device__ __forceinline__ bool chain_packed_row(const dsv_chain_args& a, int64_t row) {
  return a.p_ids != nullptr && (!a.dense_p || !(a.p_overflow && a.p_overflow[row] != 0));
}

// Entries of a packed row, clamped to [0, capacity].
__device__ __forceinline__ int chain_packed_len(const dsv_chain_args& a, int64_t row) {
  const int len = a.p_lengths[row];
  return len < 0 ? 0 : (len > a.p_cap ? a.p_cap : len);
}

// The residual's (or P's) weight at id j of a dense row: q applied per element.
__device__ __forceinline__ double chain_weight(const dsv_chain_args& a, int64_t row, int b, int step, int64_t j,
                                               bool pure, const ChainShared& sh) {
  const double P = (double)chain_dense_p(a, row, j);
  if (pure) return P;
  if (a.dense_q) {
    float q = a.dense_q[((int64_t)b * (a.T - 1) + step) * a.q_stride + j];
    q = (q >= 0.f && q <= 1.f) ? q : 0.f;
    return fmax(P - (double)q, 0.0);
  }
  double w = P;
  for (int l = 0; l < a.K; ++l)
    if (sh.qlast[l] && sh.qid[l] == j) w = fmax(P - (double)sh.qc[l], 0.0);
  return w;
}

__global__ __launch_bounds__(CH_THREADS) void k_chain(dsv_chain_args a) {
  __shared__ ChainShared sh;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int64_t V = a.vocab;
  const int T = a.T;
  int cap = a.verify_lens ? a.verify_lens[b] : T;
  cap = cap < 1 ? 1 : (cap > T ? T : cap);
  // ---- accept loop (wave 0) ----
  if (tid < WAVE && !a.p_ids && cap <= WAVE) {  // (a lane past the last step always fails)
    // dense P: every draft step's test at once, one lane a step (its token, P and q at the
    // token, its coin); the accepted length is the run of passing steps from the first
    const int step = lane + 1;
    bool ok = false;
    if (step < cap) {
      const int64_t row = chain_row(a, b, step - 1);
      const int64_t tok = a.candidates[(int64_t)b * T + step];
      const bool tok_ok = tok >= 0 && tok < V;
      const float p = tok_ok ? chain_dense_p(a, row, tok) : 0.f;
      float q = 0.f;
      if (a.dense_q) {
        if (tok_ok) q = a.dense_q[((int64_t)b * (T - 1) + step - 1) * a.q_stride + tok];
      } else {
        // the lanes holding the token, in lane order; sixteen lanes' ids and values loaded
        // together (one memory round trip per sixteen lanes, not per lane)
        const int64_t qi = ((int64_t)b * (T - 1) + step - 1) * a.K;
        for (int l0 = 0; l0 < a.K; l0 += 16) {
          int64_t id[16];
          float qv[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            const bool in = l0 + u < a.K;
            id[u] = in ? load_index(a.q_ids, a.q_ids_i64, qi + l0 + u) : -1;
            qv[u] = in ? a.q_values[qi + l0 + u] : 0.f;
          }
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (id[u] == tok) q += qv[u];
        }
      }
      const float coin = a.uniforms[(int64_t)b * (T - 1) + step - 1];
      ok = q > 0.f && q <= 1.f && coin * q < p;
    }
    const uint64_t fail = ~__ballot(ok);
    if (tid == 0) sh.acc = __ffsll((long long)fail) - 1;  // (lanes past the last step fail)
  } else if (tid < WAVE) {
    int acc = 0;
    for (int step = 1; step < cap; ++step) {
      const int64_t row = chain_row(a, b, step - 1);
      const int64_t tok = a.candidates[(int64_t)b * T + step];
      const bool tok_ok = tok >= 0 && tok < V;
      float p = 0.f;
      if (chain_packed_row(a, row)) {
        const int len = chain_packed_len(a, row);
        float part = 0.f;
        for (int i = lane; i < len; i += WAVE)
          if (a.p_ids[row * a.p_cap + i] == tok) part += a.p_values[row * a.p_cap + i];
        p = wave_sum(part);
      } else if (tok_ok) {
        p = chain_dense_p(a, row, tok);
      }
      float q = 0.f;
      if (a.dense_q) {
        if (tok_ok) q = a.dense_q[((int64_t)b * (T - 1) + step - 1) * a.q_stride + tok];
      } else {
        const int64_t qi = ((int64_t)b * (T - 1) + step - 1) * a.K;
        float part = 0.f;
        for (int l = lane; l < a.K; l += WAVE)
          if (load_index(a.q_ids, a.q_ids_i64, qi + l) == tok) part += a.q_values[qi + l];
        q = wave_sum(part);
      }
      const float coin = a.uniforms[(int64_t)b * (T - 1) + step - 1];
      if (q > 0.f && q <= 1.f && coin * q < p)
        ++acc;
      else
        break;
    }
    if (tid == 0) sh.acc = acc;
  }
  __syncthreads();
  const int acc = sh.acc;
  const bool all = acc == cap - 1;
  const int64_t row = chain_row(a, b, acc);
  if (a.overflow_read && tid < WAVE) {
    // rows 0..acc were read (the draft tests and the bonus row): any flagged overflow without a
    // dense fallback is reported
    bool bad = false;
    if (!a.dense_p && a.p_overflow)
      for (int s = lane; s <= acc; s += WAVE) bad |= a.p_overflow[chain_row(a, b, s)] != 0;
    const bool any = __ballot(bad) != 0ull;
    if (lane == 0) a.overflow_read[b] = any ? 1 : 0;
  }
  const float uf = a.uniform_final[b];
  int64_t bonus = V - 1;
  // the sparse q of the rejected step
  if (!a.dense_q) {
    const int64_t qi = ((int64_t)b * (T - 1) + acc) * a.K;
    for (int l = tid; l < QMAX; l += CH_THREADS) {
      const bool on = !all && l < a.K;
      sh.qid[l] = on ? load_index(a.q_ids, a.q_ids_i64, qi + l) : -1;
      const float q = on ? a.q_values[qi + l] : 0.f;
      sh.qc[l] = (q >= 0.f && q <= 1.f) ? q : 0.f;
      sh.qd[l] = 0.0;
    }
    __syncthreads();
    for (int l = tid; l < QMAX; l += CH_THREADS) {
      bool last = sh.qid[l] >= 0 && sh.qid[l] < V;
      for (int l2 = l + 1; l2 < a.K && last; ++l2) last = sh.qid[l2] != sh.qid[l];
      sh.qlast[l] = last;
    }
    __syncthreads();
  }
  if (chain_packed_row(a, row)) {
    // ---- packed P: entries by id (one wave) ----
    if (tid < WAVE) {
      const int len = chain_packed_len(a, row);
      const bool live = lane < len;
      const int32_t id = live ? a.p_ids[row * a.p_cap + lane] : INT_MAX;
      const float pv = live ? a.p_values[row * a.p_cap + lane] : 0.f;
      double w = pv;
      if (!all && live && !a.dense_q) {
        double at = 0.0;  // clamped q summed over the lanes with this id
        for (int l = 0; l < a.K; ++l)
          if (sh.qid[l] == (int64_t)id) at += (double)sh.qc[l];
        w = fmax((double)pv - at, 0.0);
      } else if (!all && live && a.dense_q && id >= 0 && (int64_t)id < V) {
        float q = a.dense_q[((int64_t)b * (T - 1) + acc) * a.q_stride + id];
        q = (q >= 0.f && q <= 1.f) ? q : 0.f;
        w = fmax((double)pv - (double)q, 0.0);
      }
      int rank = 0;  // position in id order
      for (int i = 0; i < len && i < WAVE; ++i) rank += __shfl(id, i, WAVE) < id;
      // weights in id order: lane `rank` of the permuted wave
      double wr = 0.0, pr = 0.0;
      int32_t idr = INT_MAX;
      for (int i = 0; i < WAVE; ++i) {
        const int ri = __shfl(rank, i, WAVE);
        const double wi = __shfl(w, i, WAVE), pi = __shfl((double)pv, i, WAVE);
        const int32_t ii = __shfl(id, i, WAVE);
        if (i < len && ri == lane) {
          wr = wi;
          pr = pi;
          idr = ii;
        }
      }
      double lo, hi;
      double mass = wave_tiles(wr, lo, hi);
      if (all || !(mass > 0.0)) mass = wave_tiles(pr, lo, hi);
      const double thr = (double)uf * mass;
      const uint64_t hit = __ballot(lane < len && idr >= 0 && (int64_t)idr < V && lo <= thr && thr < hi && hi > lo);
      if (hit) bonus = __shfl((int64_t)idr, __ffsll((long long)hit) - 1, WAVE);
      if (tid == 0) sh.bonus = bonus;
    }
    __syncthreads();
    bonus = sh.bonus;
  } else {
    // ---- dense P: tile masses, the tile holding u*mass, then its thread and id ----
    const int ntiles = (int)((V + CH_TILE - 1) / CH_TILE);
    if (!all && !a.dense_q && tid < WAVE) {  // the residual's reduction at each q id
      if (lane < a.K && sh.qlast[lane]) {
        const double P = (double)chain_dense_p(a, row, sh.qid[lane]);
        sh.qd[lane] = P - fmax(P - (double)sh.qc[lane], 0.0);
      }
    }
    __syncthreads();
    bool pure = all;
    double mass = 0.0;
    const int wid = tid / WAVE;
    // P's CH_E values of this thread in tile t (16-byte loads when the rows are aligned)
    const bool vec = a.p_stride % 4 == 0 && (uintptr_t)a.dense_p % 16 == 0;
    auto fetch = [&](int t, float (&x)[CH_E]) {
      const int64_t j0 = (int64_t)t * CH_TILE + (int64_t)tid * CH_E;
      const float* pr = a.dense_p + row * a.p_stride;
      if (vec && j0 + CH_E <= V) {
#pragma unroll
        for (int h = 0; h < CH_E / 4; ++h) {
          const float4 u = *reinterpret_cast<const float4*>(pr + j0 + 4 * h);
          x[4 * h] = u.x; x[4 * h + 1] = u.y; x[4 * h + 2] = u.z; x[4 * h + 3] = u.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < CH_E; ++e) x[e] = j0 + e < V ? pr[j0 + e] : 0.f;
      }
    };
    for (int pass = 0; pass < 2; ++pass) {
      // Tile masses.  Without a dense q the weights are P itself (the residual's reductions at
      // the sparse q ids are taken after, per tile) and each wave sums whole tiles; with a dense
      // q every wave takes its part of every tile, summed over the waves in wave order after
      // one barrier.
      const bool direct = !a.dense_q;
      const bool plain = direct && !pure;  // sparse q: P here, the q ids' reductions after
      if (direct) {
        // wave w sums whole tiles (w, w + CH_NW, ...), lane l the tile's float4s l, l + 64, ...
        // (coalesced, sixteen loads in flight); four partial sums a lane (independent chains of
        // float64 additions), then one wave reduction a tile.  RAW rows (a denominator) and the
        // others are separate instantiations: a select in the loop would compute the IEEE
        // division for every value.
        constexpr int NQ = CH_TILE / 4 / WAVE;  // float4s a lane per tile
        const float* pr = a.dense_p + row * a.p_stride;
        auto sum_tiles = [&](auto raw_tag) {
          constexpr bool RAW = decltype(raw_tag)::value;
          const float den = RAW ? a.denominator[row] : 1.f;
          for (int t = wid; t < ntiles; t += CH_NW) {
            const int64_t tlo = (int64_t)t * CH_TILE;
            double w = 0.0;
            if (vec && tlo + CH_TILE <= V) {
              float4 xb[NQ];
#pragma unroll
              for (int i = 0; i < NQ; ++i)
                xb[i] = *reinterpret_cast<const float4*>(pr + tlo + (int64_t)(i * WAVE + lane) * 4);
              double w4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
              for (int i = 0; i < NQ; ++i) {
                const float* x = reinterpret_cast<const float*>(&xb[i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) w4[e] += (double)(RAW ? x[e] / den : x[e]);
              }
              w = (w4[0] + w4[1]) + (w4[2] + w4[3]);
            } else {
              for (int64_t j = tlo + lane; j < tlo + CH_TILE && j < V; j += WAVE)
                w += (double)(RAW ? pr[j] / den : pr[j]);
            }
            w = wave_sum(w);
            if (lane == 0) sh.tile_wave[t * CH_NW] = w;
          }
        };
        if (a.denominator)
          sum_tiles(std::true_type{});
        else
          sum_tiles(std::false_type{});
      } else {
        for (int t = 0; t < ntiles; ++t) {
          const int64_t j0 = (int64_t)t * CH_TILE + (int64_t)tid * CH_E;
          double w = 0.0;
#pragma unroll
          for (int e = 0; e < CH_E; ++e)
            if (j0 + e < V) w += chain_weight(a, row, b, acc, j0 + e, pure, sh);
          w = wave_sum(w);
          if (lane == 0) sh.tile_wave[t * CH_NW + wid] = w;
        }
      }
      __syncthreads();
      for (int t = tid; t < ntiles; t += CH_THREADS) {
        double w = 0.0;
        if (direct)
          w = sh.tile_wave[t * CH_NW];
        else
          for (int i = 0; i < CH_NW; ++i) w += sh.tile_wave[t * CH_NW + i];
        if (plain)  // sparse q: the tile's reductions at its q ids
          for (int l = 0; l < a.K; ++l)
            if (sh.qlast[l] && sh.qid[l] / CH_TILE == t) w -= sh.qd[l];
        sh.tile_mass[t] = w;
      }
      __syncthreads();
      if (ntiles <= WAVE) {  // the total by a wave scan over the tiles (lanes hold tiles)
        if (tid < WAVE) {
          double lo, hi;
          const double tot = wave_tiles(lane < ntiles ? sh.tile_mass[lane] : 0.0, lo, hi);
          if (lane == 0) sh.mass = tot;
        }
        __syncthreads();
        mass = sh.mass;
      } else {
        mass = 0.0;
        for (int t = 0; t < ntiles; ++t) mass += sh.tile_mass[t];
      }
      if (pure || mass > 0.0) break;
      __syncthreads();  // (the second pass rewrites the tiles' parts)
      pure = true;  // the residual has no mass: draw from P
    }
    __syncthreads();
    const double thr = (double)uf * mass;
    if (ntiles <= WAVE && tid < WAVE) {
      // the first tile with mass whose interval (the same scan as the total) ends past thr
      const double m = lane < ntiles ? sh.tile_mass[lane] : 0.0;
      double lo, hi;
      wave_tiles(m, lo, hi);
      uint64_t hit = __ballot(lane < ntiles && m > 0.0 && thr < hi);
      if (!hit) {  // rounding: the last tile with mass
        const uint64_t pos = __ballot(lane < ntiles && m > 0.0);
        hit = pos ? 1ull << (63 - __clzll((long long)pos)) : 0ull;
      }
      const int tile = hit ? __ffsll((long long)hit) - 1 : -1;
      const double before = readlane_at(lo, tile >= 0 ? tile : 0);
      if (lane == 0) {
        sh.tile = tile;
        sh.tile_lo = tile >= 0 ? before : 0.0;
        sh.thr = thr;
        sh.pure = pure ? 1 : 0;
        sh.pick_thread = -1;
        sh.bonus = V - 1;
      }
    } else if (ntiles > WAVE && tid == 0) {
      double before = 0.0;
      int tile = -1, last = -1;
      for (int t = 0; t < ntiles; ++t) {
        const double m = sh.tile_mass[t];
        if (m > 0.0) last = t;
        if (tile < 0 && m > 0.0 && before + m > thr) tile = t;
        if (tile < 0) before += m;
      }
      if (tile < 0 && last >= 0) {  // rounding: the last tile with mass
        tile = last;
        before = 0.0;
        for (int t = 0; t < last; ++t) before += sh.tile_mass[t];
      }
      sh.tile = tile;
      sh.tile_lo = before;
      sh.thr = thr;
      sh.pure = pure ? 1 : 0;
      sh.pick_thread = -1;
      sh.bonus = V - 1;
    }
    __syncthreads();
    const int tile = sh.tile;
    if (tile >= 0) {
      const bool pu = sh.pure != 0;
      const int64_t j0 = (int64_t)tile * CH_TILE + (int64_t)tid * CH_E;
      double w[CH_E];
      double wt = 0.0;
      if (!a.dense_q) {
        // P from one vector load, then the residual at the sparse q ids inside this thread's
        // eight (the last lane with an id carries its q)
        float x[CH_E];
        fetch(tile, x);
        if (a.denominator) {  // (a branch: a select would divide every value)
          const float den = a.denominator[row];
#pragma unroll
          for (int e = 0; e < CH_E; ++e) x[e] = x[e] / den;
        }
#pragma unroll
        for (int e = 0; e < CH_E; ++e) w[e] = j0 + e < V ? (double)x[e] : 0.0;
        if (!pu)
          for (int l = 0; l < a.K; ++l) {
            const uint64_t o = (uint64_t)(sh.qid[l] - j0);
            if (sh.qlast[l] && o < (uint64_t)CH_E) {
#pragma unroll
              for (int e = 0; e < CH_E; ++e)
                if ((uint64_t)e == o) w[e] = fmax(w[e] - (double)sh.qc[l], 0.0);
            }
          }
#pragma unroll
        for (int e = 0; e < CH_E; ++e) wt += w[e];
      } else {
#pragma unroll
        for (int e = 0; e < CH_E; ++e) {
          w[e] = j0 + e < V ? chain_weight(a, row, b, acc, j0 + e, pu, sh) : 0.0;
          wt += w[e];
        }
      }
      double tlo, thi;
      block_tiles<CH_NW>(wt, sh.red_d, tlo, thi);
      const double base = sh.tile_lo;
      if (wt > 0.0 && base + tlo <= sh.thr && sh.thr < base + thi) sh.pick_thread = tid;
      __syncthreads();
      int pt = sh.pick_thread;
      if (pt < 0) {  // rounding: the last thread with mass
        const uint64_t lp = block_max_u64<CH_NW>(wt > 0.0 ? (uint64_t)tid + 1 : 0ull,
                                                 reinterpret_cast<uint64_t*>(sh.red_d));
        pt = lp ? (int)lp - 1 : -1;
      }
      if (tid == pt) {
        double c = base + tlo;
        int64_t pick = -1, last = -1;
#pragma unroll
        for (int e = 0; e < CH_E; ++e) {
          if (w[e] > 0.0) {
            last = j0 + e;
            if (pick < 0 && c + w[e] > sh.thr) pick = j0 + e;
          }
          c += w[e];
        }
        sh.bonus = pick >= 0 ? pick : last;
      }
      __syncthreads();
      bonus = sh.bonus;
    }
  }
  // ---- outputs ----
  for (int i = tid; i < T; i += CH_THREADS) {
    int64_t val = 0;
    if (i < acc)
      val = a.candidates[(int64_t)b * T + i + 1];
    else if (i == acc)
      val = bonus;
    a.output[(int64_t)b * T + i] = val;
  }
  if (tid == 0) {
    a.accept[b] = acc;
    a.commit[b] = acc + 1;
    a.bonus[b] = bonus;
    a.new_seq[b] = a.prefix_lens[b] + acc + 1;
  }
}

// ---------------------------------------------------------------------------------------
// Draft-side K-lane chain (kernels/dspine.py:616-674): one wave per request walks its T-1 rows
// of the [K, K] table; lanes are the K candidates.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(WAVE) void k_sample_chain(const float* table, int32_t K, int32_t tm1,
                                                      const float* inv_temp, const int32_t* top_k,
                                                      const float* top_p, const float* min_p, const int32_t* greedy,
                                                      const float* u, const int64_t* cand, const int64_t* greedy_tok,
                                                      int64_t* out_tok, float* out_q, float* confidence) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const bool live = lane < K;
  const float inv_t = inv_temp[b];
  const int32_t tk = top_k[b];
  const float tp = top_p[b];
  const float mp = min_p[b];
  const bool gr = greedy[b] != 0;
  int sender = 0;
  for (int i = 0; i < tm1; ++i) {
    const int64_t n = (int64_t)b * tm1 + i;
    const float score = live ? table[(n * K + sender) * K + lane] * inv_t : -INFINITY;
    float mx = score;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, WAVE));
    const float mass = live ? expf(score - mx) : 0.f;
    float tot = mass;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, WAVE);
    const float p = live ? mass / tot : -1.f;
    float pmax = p;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) pmax = fmaxf(pmax, __shfl_xor(pmax, o, WAVE));
    if (confidence && !gr && lane == 0) confidence[n] = pmax;
    // rank and mass ahead (ties: lower lane first)
    int rank = 0;
    float before = 0.f;
    for (int d = 0; d < K; ++d) {
      const float pd = __shfl(p, d, WAVE);
      const bool ahead = pd > p || (pd == p && d < lane);
      rank += ahead;
      before += ahead ? pd : 0.f;
    }
    const bool keep = live && rank < tk && before <= tp && p >= mp * pmax;
    const float w = keep ? p : 0.f;
    float ws = w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ws += __shfl_xor(ws, o, WAVE);
    const float q = live ? w / ws : 0.f;
    // inclusive prefix of q in lane order
    float cdf = q;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
      const float t = __shfl_up(cdf, o, WAVE);
      if (lane >= o) cdf += t;
    }
    const float total = __shfl(cdf, K - 1, WAVE);
    const float threshold = u[n] * total;
    int choice = __popcll(__ballot(live && cdf <= threshold));
    const uint64_t kept = __ballot(keep);
    const int last = kept ? 63 - __clzll((long long)kept) : 0;
    choice = choice < last ? choice : last;
    const int64_t cl = live ? cand[n * K + lane] : 0;
    const int64_t sampled = __shfl(cl, choice, WAVE);
    const int64_t gtok = greedy_tok[n];
    if (lane == 0) out_tok[n] = gr ? gtok : sampled;
    if (live) out_q[n * K + lane] = gr ? (cl == gtok ? 1.f : 0.f) : q;
    sender = choice;
  }
}


// ---------------------------------------------------------------------------------------
// Sparse joint target (sampling/sparse/target.py:22-66, CPU form :156-178).  One wave per row
// over the row's top-W of P (values descending, ids; W <= 64): keep p > 0, p >= p[k-1] and the
// nucleus (mass of strictly larger p < top_p, or top_p >= 1); the kept ids ascending with
// p / sum(kept) fill [capacity] slots (then -1 / 0); overflow = count > capacity.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(WAVE) void k_pack_joint(const float* top_vals, const int64_t* top_ids, int32_t W,
                                                    const int32_t* top_ks, const float* top_ps, int32_t capacity,
                                                    int32_t* ids, float* values, int32_t* lengths,
                                                    int32_t* overflow) {
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  const bool live = lane < W;
  const float p = live ? top_vals[r * W + lane] : 0.f;
  const int64_t id = live ? top_ids[r * W + lane] : INT64_MAX;
  int k = top_ks[r];
  k = k < 1 ? 1 : (k > W ? W : k);
  const float threshold = __shfl(p, k - 1, WAVE);
  const float tp = top_ps[r];
  float higher = 0.f;  // mass of strictly larger p, in rank order
  for (int j = 0; j < W; ++j) {
    const float pj = __shfl(p, j, WAVE);
    higher += pj > p ? pj : 0.f;
  }
  const bool keep = live && p > 0.f && p >= threshold && (higher < tp || tp >= 1.f);
  const uint64_t kept = __ballot(keep);
  const int count = __popcll(kept);
  float total = 0.f;  // the kept mass, summed in rank order
  for (int j = 0; j < W; ++j) {
    const float pj = __shfl(p, j, WAVE);
    total += ((kept >> j) & 1ull) ? pj : 0.f;
  }
  int rank = 0;  // position among the kept ids in ascending id order
  for (int j = 0; j < W; ++j) rank += ((kept >> j) & 1ull) && __shfl(id, j, WAVE) < id;
  if (keep && rank < capacity) {
    ids[r * capacity + rank] = (int32_t)id;
    values[r * capacity + rank] = p / total;
  }
  for (int i = count + lane; i < capacity; i += WAVE) {
    ids[r * capacity + i] = -1;
    values[r * capacity + i] = 0.f;
  }
  if (lane == 0) {
    lengths[r] = count < capacity ? count : capacity;
    overflow[r] = count > capacity ? 1 : 0;
  }
}

// Overflow rows of the sparse joint target: P[r] = p * (p >= p[k-1]) / sum, in place.
__global__ __launch_bounds__(CMP_THREADS) void k_overflow_dense(const float* top_vals, int32_t W,
                                                               const int32_t* top_ks, const int32_t* overflow,
                                                               float* P, int64_t vocab, int64_t p_stride) {
  constexpr int NW = CMP_THREADS / WAVE;
  __shared__ double red[NW];
  const int64_t r = blockIdx.x;
  if (overflow[r] == 0) return;
  int k = top_ks[r];
  k = k < 1 ? 1 : (k > W ? W : k);
  const float threshold = top_vals[r * W + k - 1];
  float* row = P + r * p_stride;
  double s = 0.0;
  for (int64_t j = threadIdx.x; j < vocab; j += CMP_THREADS) {
    const float x = row[j];
    s += x >= threshold ? (double)x : 0.0;
  }
  const float total = (float)block_sum<NW>(s, red);
  for (int64_t j = threadIdx.x; j < vocab; j += CMP_THREADS) {
    const float x = row[j];
    row[j] = x >= threshold ? x / total : 0.f;
  }
}

}  // namespace dsv

// =========================================================================================
// Host entry points
// =========================================================================================
using namespace dsv;

static dim3 row_grid(int64_t rows, int64_t vocab) {
  int64_t bx = (vocab + ADJ_THREADS * 4 - 1) / (ADJ_THREADS * 4);
  if (bx > 64) bx = 64;
  if (bx < 1) bx = 1;
  return dim3((unsigned)bx, (unsigned)rows);
}

extern "C" int dsv_adjust_logits(void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                                 const int64_t* row_to_request, int32_t rows_per_request, int64_t requests,
                                 int32_t op, const float* values, int64_t values_stride, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!logits || !values) DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_logits: null pointer");
  if (logits_dtype != DSV_F32 && logits_dtype != DSV_BF16)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_logits: logits must be float32 or bfloat16");
  if (op != DSV_ADJ_ADD && op != DSV_ADJ_SCALE) DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_logits: unknown op %d", op);
  if (rows < 0 || vocab < 1 || row_stride < vocab || values_stride < vocab || requests < 1)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_logits: invalid shape");
  if (!row_to_request && (rows_per_request < 1 || rows > requests * rows_per_request))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_logits: %lld rows do not fit %lld requests x %d rows",
             (long long)rows, (long long)requests, rows_per_request);
  if (rows == 0) return DSV_OK;
  if (rows > 65535) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_adjust_logits: at most 65535 rows per call");
  const int64_t esize = logits_dtype == DSV_BF16 ? 2 : 4;
  const bool vec = (uintptr_t)logits % 16 == 0 && (row_stride * esize) % 16 == 0 && (uintptr_t)values % 16 == 0 &&
                   values_stride % 4 == 0;
  if (vec && logits_dtype == DSV_BF16 && !row_to_request && rows_per_request > 1) {
    const int64_t bx = (vocab + ADJ_THREADS * ADJ_VEC - 1) / (ADJ_THREADS * ADJ_VEC);
    const int64_t nreq = (rows + rows_per_request - 1) / rows_per_request;
    // (the op as a template argument: a run-time select would compute the division of every value)
    const dim3 grid((unsigned)bx, (unsigned)nreq);
    if (op == DSV_ADJ_ADD)
      hipLaunchKernelGGL((k_adjust_req<uint16_t, DSV_ADJ_ADD>), grid, dim3(ADJ_THREADS), 0, stream, (uint16_t*)logits,
                         vocab, row_stride, rows, rows_per_request, values, values_stride);
    else
      hipLaunchKernelGGL((k_adjust_req<uint16_t, DSV_ADJ_SCALE>), grid, dim3(ADJ_THREADS), 0, stream,
                         (uint16_t*)logits, vocab, row_stride, rows, rows_per_request, values, values_stride);
  } else if (vec) {
    int64_t bx = (vocab + ADJ_THREADS * ADJ_VEC - 1) / (ADJ_THREADS * ADJ_VEC);
    if (bx > 64) bx = 64;
    const dim3 grid((unsigned)bx, (unsigned)((rows + ADJ_ROWS - 1) / ADJ_ROWS));
    if (logits_dtype == DSV_BF16 && op == DSV_ADJ_ADD)
      hipLaunchKernelGGL((k_adjust_vec<uint16_t, DSV_ADJ_ADD>), grid, dim3(ADJ_THREADS), 0, stream, (uint16_t*)logits,
                         vocab, row_stride, rows, row_to_request, rows_per_request, values, values_stride);
    else if (logits_dtype == DSV_BF16)
      hipLaunchKernelGGL((k_adjust_vec<uint16_t, DSV_ADJ_SCALE>), grid, dim3(ADJ_THREADS), 0, stream,
                         (uint16_t*)logits, vocab, row_stride, rows, row_to_request, rows_per_request, values,
                         values_stride);
    else if (op == DSV_ADJ_ADD)
      hipLaunchKernelGGL((k_adjust_vec<float, DSV_ADJ_ADD>), grid, dim3(ADJ_THREADS), 0, stream, (float*)logits, vocab,
                         row_stride, rows, row_to_request, rows_per_request, values, values_stride);
    else
      hipLaunchKernelGGL((k_adjust_vec<float, DSV_ADJ_SCALE>), grid, dim3(ADJ_THREADS), 0, stream, (float*)logits,
                         vocab, row_stride, rows, row_to_request, rows_per_request, values, values_stride);
  } else {
    const dim3 grid = row_grid(rows, vocab);
    if (logits_dtype == DSV_BF16)
      hipLaunchKernelGGL(k_adjust<uint16_t>, grid, dim3(ADJ_THREADS), 0, stream, (uint16_t*)logits, vocab,
                         row_stride, row_to_request, rows_per_request, op, values, values_stride);
    else
      hipLaunchKernelGGL(k_adjust<float>, grid, dim3(ADJ_THREADS), 0, stream, (float*)logits, vocab, row_stride,
                         row_to_request, rows_per_request, op, values, values_stride);
  }
  DSV_CHECK_LAUNCH("dsv_adjust_logits");
  return DSV_OK;
}

extern "C" int dsv_adjust_history(void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                                  const int64_t* row_to_request, int32_t rows_per_request, int64_t requests,
                                  const int32_t* hist_ids, int32_t hist_len, const float* presence,
                                  const float* repetition, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!logits || (hist_len > 0 && !hist_ids)) DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_history: null pointer");
  if (logits_dtype != DSV_F32 && logits_dtype != DSV_BF16)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_history: logits must be float32 or bfloat16");
  if (rows < 0 || vocab < 1 || row_stride < vocab || requests < 1 || hist_len < 0)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_history: invalid shape");
  if (!row_to_request && (rows_per_request < 1 || rows > requests * rows_per_request))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_adjust_history: rows do not fit the requests");
  const size_t lds = (size_t)((vocab + 31) / 32) * 4;
  if (lds > 64 * 1024) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_adjust_history: vocab too large for the LDS bitmap");
  if (rows == 0 || hist_len == 0 || (!presence && !repetition)) return DSV_OK;
  if (logits_dtype == DSV_BF16) {
    (void)hipFuncSetAttribute((const void*)k_adjust_history<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    hipLaunchKernelGGL(k_adjust_history<uint16_t>, dim3((unsigned)rows), dim3(ADJ_THREADS), lds, stream,
                       (uint16_t*)logits, vocab, row_stride, row_to_request, rows_per_request, hist_ids, hist_len,
                       presence, repetition);
  } else {
    (void)hipFuncSetAttribute((const void*)k_adjust_history<float>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    hipLaunchKernelGGL(k_adjust_history<float>, dim3((unsigned)rows), dim3(ADJ_THREADS), lds, stream, (float*)logits,
                       vocab, row_stride, row_to_request, rows_per_request, hist_ids, hist_len, presence, repetition);
  }
  DSV_CHECK_LAUNCH("dsv_adjust_history");
  return DSV_OK;
}

extern "C" int dsv_logits_padding(void* out, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                                  dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!out) DSV_FAIL(DSV_ERR_INVALID, "dsv_logits_padding: null pointer");
  if (dtype != DSV_F32 && dtype != DSV_BF16) DSV_FAIL(DSV_ERR_INVALID, "dsv_logits_padding: float32 or bfloat16");
  if (rows < 0 || vocab < 1 || row_stride < vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_logits_padding: invalid shape");
  if (rows == 0) return DSV_OK;
  if (rows > 65535) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_logits_padding: at most 65535 rows per call");
  const dim3 grid = row_grid(rows, vocab);
  if (dtype == DSV_BF16)
    hipLaunchKernelGGL(k_padding<uint16_t>, grid, dim3(ADJ_THREADS), 0, stream, (uint16_t*)out, vocab, row_stride);
  else
    hipLaunchKernelGGL(k_padding<float>, grid, dim3(ADJ_THREADS), 0, stream, (float*)out, vocab, row_stride);
  DSV_CHECK_LAUNCH("dsv_logits_padding");
  return DSV_OK;
}

extern "C" int dsv_window_index(const void* qo_indptr, int32_t qo_i64, int32_t bs, int32_t T, int64_t* out,
                                int64_t total, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!qo_indptr || !out) DSV_FAIL(DSV_ERR_INVALID, "dsv_window_index: null pointer");
  if (bs < 0 || T < 1 || total < 0) DSV_FAIL(DSV_ERR_INVALID, "dsv_window_index: invalid shape");
  if (bs == 0 || total == 0) return DSV_OK;
  hipLaunchKernelGGL(k_window_index, dim3((unsigned)bs), dim3(64), 0, stream, qo_indptr, qo_i64, T, out, total);
  DSV_CHECK_LAUNCH("dsv_window_index");
  return DSV_OK;
}

extern "C" int dsv_compress(const float* p, int64_t rows, int64_t vocab, int64_t row_stride, int32_t capacity,
                            int32_t* ids, float* values, int32_t* lengths, int32_t* overflow, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!p || !ids || !values || !lengths || !overflow) DSV_FAIL(DSV_ERR_INVALID, "dsv_compress: null pointer");
  if (rows < 0 || vocab < 1 || row_stride < vocab || capacity < 1)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_compress: invalid shape");
  if (vocab >= (1ll << 31)) DSV_FAIL(DSV_ERR_INVALID, "dsv_compress: vocab must be < 2^31");
  if (rows == 0) return DSV_OK;
  hipLaunchKernelGGL(k_compress, dim3((unsigned)rows), dim3(CMP_THREADS), 0, stream, p, vocab, row_stride, capacity,
                     ids, values, lengths, overflow);
  DSV_CHECK_LAUNCH("dsv_compress");
  return DSV_OK;
}

extern "C" int dsv_accept_chain(const dsv_chain_args* args, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: null arguments");
  const dsv_chain_args& a = *args;
  if (a.bs < 0 || a.T < 2 || a.vocab < 1) DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: invalid shape");
  if (a.vocab > (int64_t)CH_TILES_MAX * CH_TILE)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_accept_chain: vocab %lld > %d", (long long)a.vocab, CH_TILES_MAX * CH_TILE);
  if (!a.candidates || !a.uniforms || !a.uniform_final || !a.prefix_lens || !a.accept || !a.commit || !a.bonus ||
      !a.output || !a.new_seq)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: required pointer is null");
  if (!a.dense_p && !a.p_ids) DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: no target distribution");
  if (a.dense_p && a.p_stride < a.vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: dense P row stride");
  if (a.p_ids && (!a.p_values || !a.p_lengths || a.p_cap < 1))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: packed P needs ids, values, lengths and a capacity");
  if (a.p_ids && a.p_cap > CH_PACK_MAX)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_accept_chain: packed capacity %d > %d", a.p_cap, CH_PACK_MAX);
  if (!a.dense_q && (!a.q_ids || !a.q_values || a.K < 1 || a.K > QMAX))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: sparse q needs ids, values and 1 <= K <= %d", QMAX);
  if (a.dense_q && a.q_stride < a.vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_accept_chain: dense q row stride");
  if (a.bs == 0) return DSV_OK;
  hipLaunchKernelGGL(k_chain, dim3((unsigned)a.bs), dim3(CH_THREADS), 0, stream, a);
  DSV_CHECK_LAUNCH("dsv_accept_chain");
  return DSV_OK;
}

extern "C" int dsv_sample_chain(const float* table, int64_t n, int32_t K, int32_t block_size, const float* inv_temp,
                                const int32_t* top_k, const float* top_p, const float* min_p, const int32_t* greedy,
                                const float* u, const int64_t* cand, const int64_t* greedy_tok, int64_t* out_tok,
                                float* out_q, float* confidence, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!table || !inv_temp || !top_k || !top_p || !min_p || !greedy || !u || !cand || !greedy_tok || !out_tok ||
      !out_q)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_sample_chain: null pointer");
  if (K < 1 || K > WAVE) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_sample_chain: K=%d outside [1, %d]", K, WAVE);
  if (block_size < 2 || n < 0 || n % (block_size - 1))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_sample_chain: %lld rows are not whole chains of %d", (long long)n,
             block_size - 1);
  const int64_t bs = n / (block_size - 1);
  if (bs == 0) return DSV_OK;
  if (bs > 2147483647ll) DSV_FAIL(DSV_ERR_INVALID, "dsv_sample_chain: too many chains");
  hipLaunchKernelGGL(k_sample_chain, dim3((unsigned)bs), dim3(WAVE), 0, stream, table, K, block_size - 1, inv_temp,
                     top_k, top_p, min_p, greedy, u, cand, greedy_tok, out_tok, out_q, confidence);
  DSV_CHECK_LAUNCH("dsv_sample_chain");
  return DSV_OK;
}

extern "C" int dsv_pack_joint(const float* top_vals, const int64_t* top_ids, int64_t rows, int32_t W,
                              const int32_t* top_ks, const float* top_ps, int32_t capacity, int32_t* ids,
                              float* values, int32_t* lengths, int32_t* overflow, float* P, int64_t vocab,
                              int64_t p_stride, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!top_vals || !top_ids || !top_ks || !top_ps || !ids || !values || !lengths || !overflow)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_pack_joint: null pointer");
  if (rows < 0 || W < 1 || capacity < 1 || W > capacity + 1)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_pack_joint: invalid shape (W=%d, capacity=%d)", W, capacity);
  if (W > WAVE) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_pack_joint: W=%d > %d", W, WAVE);
  if (P && (vocab < W || p_stride < vocab)) DSV_FAIL(DSV_ERR_INVALID, "dsv_pack_joint: invalid dense P shape");
  if (rows == 0) return DSV_OK;
  if (rows > 2147483647ll) DSV_FAIL(DSV_ERR_INVALID, "dsv_pack_joint: too many rows");
  hipLaunchKernelGGL(k_pack_joint, dim3((unsigned)rows), dim3(WAVE), 0, stream, top_vals, top_ids, W, top_ks, top_ps,
                     capacity, ids, values, lengths, overflow);
  DSV_CHECK_LAUNCH("dsv_pack_joint");
  if (P) {
    hipLaunchKernelGGL(k_overflow_dense, dim3((unsigned)rows), dim3(CMP_THREADS), 0, stream, top_vals, W, top_ks,
                       overflow, P, vocab, p_stride);
    DSV_CHECK_LAUNCH("dsv_pack_joint");
  }
  return DSV_OK;
}
