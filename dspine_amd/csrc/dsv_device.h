// Device building blocks of the verification kernels: element access, keys, penalties,
// candidate selection, and the shared workspace records.
#pragma once
#include <limits.h>

#include "dsv_common.h"

namespace dsv {

enum RowMode { M_SKIP = 0, M_GREEDY = 1, M_LIST = 2, M_UNF = 3, M_HIST = 4 };

// Per-row result consumed by the rejection walk and the bonus draw.
struct RowSum {
  int32_t mode;
  int32_t argmax;   // first maximal id of the adjusted row
  uint32_t kmax;    // key of the maximum
  uint32_t vcut;    // HIST: kept iff key > vcut or (key == vcut and tie rank < ktie)
  int32_t ktie;
  int32_t nlist;    // LIST/GREEDY: support entries
  float m_f;        // fp32(max / T)
  float invZ;       // fp32(1 / Z)
  float S_f;        // normaliser of the filtered row (1 when unfiltered)
  float p_draft;    // P at this row's draft token
  int32_t flags;
  int32_t norm;     // UNF rows: 1 when P = p / S_f (filter on, nothing cut)
  double Z;
  double S_kept;
};
static_assert(sizeof(RowSum) == 64, "RowSum layout");

struct ListEntry {
  int32_t id;
  float P;
};

// Per-chunk partial statistics of the chunked row pass.
struct ChunkStat {
  float m;        // chunk max of the adjusted values (-inf when empty)
  int32_t arg;    // first id attaining it
  double s;       // sum exp((x - m) / T) over the chunk
  int32_t ncand;  // candidates written (LIST)
  int32_t tieq;   // nucleus rows: values of the chunk with the draft token's key and a lower id
  uint32_t wlo;   // nucleus rows: lowest key of the chunk's value-count window (WIN_EMPTY: none)
  uint32_t kx;    // nucleus rows: largest key below the window (0: none; KX_UNKNOWN: not tracked)
  float xtok;     // softmax rows: the draft token's adjusted value, in the chunk that holds it
  int32_t pad;
};
static_assert(sizeof(ChunkStat) == 40, "ChunkStat layout");


constexpr int CT = 256;              // threads of a chunk workgroup
constexpr int CV_MAX = 12;           // most 16-byte vectors a thread holds of a chunk (float32 rows)
constexpr int CAND_CAP = 512;        // LDS candidate buffer of a chunk (> largest k)
constexpr int TOPK_MAX = 256;        // largest k of the top-k entry point
constexpr int NUC_THREADS = 512;     // full-histogram nucleus workgroup
constexpr int HIST_WORDS = 32768;    // 65536 16-bit counters
constexpr int NUC_SLICE = 65528;     // values per 16-bit histogram pass (no counter can wrap)
constexpr int HWIN = 4096;           // keys of a chunk's value-count window (nucleus rows)
constexpr uint32_t WIN_EMPTY = 0x10000u;
constexpr uint32_t KX_UNKNOWN = 0xFFFFFFFFu;  // ChunkStat::kx when the chunk did not track it
constexpr int STAGE_VECS = 256;      // list rows: vectors (those reaching the admission bound) the LDS stage holds
constexpr int WHITV = 64;            // LDS slots of a wave for vectors holding history hits
constexpr int NCHK = 32;             // most chunks a row may have (per-row chunk arrays)
constexpr int BCT = 256;             // threads of the bonus / finalize kernels
constexpr int QMAX = 64;             // largest supported sparse-q width K
constexpr int FLAG_FULL_HIST = 2;    // nucleus row whose cut needs the full value histogram
constexpr int FLAG_SCAN_DRAW = 4;    // dense row whose bonus draw k_final plans from a scan of every chunk
constexpr int FLAG_TIES_COUNTED = 8; // full-histogram row whose chunks' counts of cut-key values are in rties
constexpr int SJ_CAP = 32;           // packed capacity of the sparse joint target (sampling/target.py:84-87)

template <int DT>
struct Elems {
  static constexpr int n = DT == DSV_BF16 ? 8 : 4;    // elements per 16-byte vector
  static constexpr int cv = DT == DSV_BF16 ? 10 : 12;  // 16-byte vectors per thread per chunk
  static constexpr int chunk = CT * cv * n;
};
static_assert(Elems<DSV_F32>::cv <= CV_MAX && Elems<DSV_BF16>::cv <= CV_MAX, "CV_MAX bounds both");

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ int req_cap(const dsv_verify_args& a, int b) {
  int cap = a.verify_lens ? a.verify_lens[b] : a.T;
  return cap < 1 ? 1 : (cap > a.T ? a.T : cap);
}

// Row r -> (request b, position s); false when r is not a verified row.
__device__ __forceinline__ bool row_request(const dsv_verify_args& a, int64_t r, int& b, int& s) {
  if (a.row_offsets == nullptr) {
    // (rows < 2^31: a 32-bit division)
    b = (int)((uint32_t)r / (uint32_t)a.T);
    s = (int)((uint32_t)r - (uint32_t)b * (uint32_t)a.T);
  } else {
    if (load_index(a.row_offsets, a.row_offsets_i64, 0) > r) return false;
    int lo = 0, hi = a.bs - 1;
    while (lo < hi) {  // largest b with offset[b] <= r
      const int mid = (lo + hi + 1) >> 1;
      if (load_index(a.row_offsets, a.row_offsets_i64, mid) <= r)
        lo = mid;
      else
        hi = mid - 1;
    }
    b = lo;
    s = (int)(r - load_index(a.row_offsets, a.row_offsets_i64, b));
  }
  if (b < 0 || b >= a.bs) return false;
  return s >= 0 && s < req_cap(a, b);
}

__device__ __forceinline__ int64_t request_row0(const dsv_verify_args& a, int b) {
  return a.row_offsets ? load_index(a.row_offsets, a.row_offsets_i64, b) : (int64_t)b * a.T;
}

// Which pass a row needs.  Rows of filtered requests whose top-k is off, whose top-p is >= 1
// and without min-p are unfiltered in effect (only the renormalisation remains): M_UNF with
// norm.  Nucleus rows (a cut that is neither a short top-k nor absent) need M_HIST.
__device__ __forceinline__ int row_mode(const dsv_verify_args& a, int b, int force_greedy) {
  if (force_greedy) return M_GREEDY;
  const int k = a.top_ks[b];
  if (a.any_greedy && k <= 1) return M_GREEDY;
  if (a.sparse_joint) return M_LIST;  // (every top-k <= SJ_CAP; the filter applies whatever the flags)
  if (!a.filter) return M_UNF;
  if (k <= DSV_LIST_K) return M_LIST;
  const float mp = (a.need_min_p && a.min_ps) ? a.min_ps[b] : 0.f;
  if (a.top_ps[b] >= 1.f && mp <= 0.f && (int64_t)k >= a.vocab) return M_UNF;
  return M_HIST;
}

// ---------------------------------------------------------------------------------------
// Elements
// ---------------------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ uint32_t key_of(float x) {
  if constexpr (DT == DSV_BF16)
    return bf16_key(__float_as_uint(x) >> 16);
  else
    return f32_key(x);
}
template <int DT>
__device__ __forceinline__ float value_of_key(uint32_t k) {
  if constexpr (DT == DSV_BF16)
    return bf16_key_to_f32(k);
  else
    return key_to_f32(k);
}
template <int DT>
__device__ __forceinline__ float load_elem(const char* rowp, int64_t j) {
  if constexpr (DT == DSV_BF16)
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(rowp)[j]);
  else
    return reinterpret_cast<const float*>(rowp)[j];
}

// Element e of a 16-byte vector.
template <int DT>
__device__ __forceinline__ float vec_elem(const uint4& v, int e) {
  const uint32_t w = e < (DT == DSV_BF16 ? 2 : 1) ? v.x
                     : e < (DT == DSV_BF16 ? 4 : 2) ? v.y
                     : e < (DT == DSV_BF16 ? 6 : 3) ? v.z
                                                    : v.w;
  if constexpr (DT == DSV_BF16)
    return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  else
    return __uint_as_float(w);
}

// The 16 bits of bf16 element e (0..7, a compile-time index) of a 16-byte vector.
__device__ __forceinline__ uint32_t bf16_bits(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return (e & 1) ? w >> 16 : w & 0xffffu;
}

typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
constexpr uint32_t FILL_BF16 = 0xFF80FF80u;  // two bf16 -inf
constexpr uint32_t FILL_F32 = 0xFF800000u;   // float -inf

// Load 16-byte vector vi of a row (elements [vi*n, vi*n+n)), -inf past `hi` (element index).
template <int DT>
__device__ __forceinline__ uint4 load_vec(const char* rowp, int64_t vi, int64_t hi, bool aligned) {
  constexpr int n = Elems<DT>::n;
  const int64_t j0 = vi * n;
  const uint32_t fill = DT == DSV_BF16 ? FILL_BF16 : FILL_F32;
  if (aligned && j0 + n <= hi) {
    const v4u_t t = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(rowp) + vi);
    return make_uint4(t.x, t.y, t.z, t.w);
  }
  uint32_t w[4] = {fill, fill, fill, fill};
  if (j0 < hi) {
    if constexpr (DT == DSV_BF16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(rowp);
      for (int e = 0; e < 8; ++e) {
        const uint32_t b = (j0 + e < hi) ? p[j0 + e] : 0xFF80u;
        w[e >> 1] = (e & 1) ? ((w[e >> 1] & 0xffffu) | (b << 16)) : ((w[e >> 1] & 0xffff0000u) | b);
      }
    } else {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(rowp);
      for (int e = 0; e < 4; ++e) w[e] = (j0 + e < hi) ? p[j0 + e] : FILL_F32;
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// An empty asm that claims to rewrite the registers: values unpacked from them before the
// fence cannot be reused after it, so each pass unpacks its elements again instead of the
// compiler keeping every unpacked element alive across passes.
template <int N>
__device__ __forceinline__ void reg_fence(uint4 (&v)[N]) {
#pragma unroll
  for (int u = 0; u < N; ++u) asm volatile("" : "+v"(v[u].x), "+v"(v[u].y), "+v"(v[u].z), "+v"(v[u].w));
}

// The same for one vector: the elements of a vector are unpacked after the fence, one
// vector at a time.
__device__ __forceinline__ void reg_fence1(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}
// ... and after `acc` (a running result of the previous vectors) is final, which keeps the
// unpacking of the next vector from being scheduled ahead of the current one.
__device__ __forceinline__ void reg_fence1(uint4& v, float& acc) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w), "+v"(acc));
}
__device__ __forceinline__ void reg_fence1(uint4& v, int& acc) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w), "+v"(acc));
}
// Orders `acc` after the vector without redefining the vector (for passes inside a branch,
// where a redefinition would make the compiler copy every vector at the join).
__device__ __forceinline__ void order_after(const uint4& v, int& acc) {
  asm volatile("" : "+v"(acc) : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}

// Two 16-bit differences a - b, each wrapping modulo 2^16.
__device__ __forceinline__ uint32_t sub_u16x2(uint32_t a, uint32_t b) {
  typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}

// The J-th largest (1 <= J <= 64) of the wave's BITS-bit keys: a radix select on ballots.
template <int BITS>
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t k, int J) {
  uint32_t pre = 0u;
#pragma unroll
  for (int bit = BITS - 1; bit >= 0; --bit) {
    const uint32_t cand = pre | (1u << bit);
    if (__popcll(__ballot(k >= cand)) >= J) pre = cand;
  }
  return pre;
}

// The smallest key k in [lo, hi] with pred(k), for a pred that is false and then true as the key
// grows (hi is taken to hold it, untested): a 64-way search, one key a lane a round -- three rounds
// for 16-bit keys -- where a bisection by one thread takes sixteen dependent steps.  Wave-wide
// (every lane active); the result in every lane.
template <class F>
__device__ __forceinline__ uint32_t wave_first_key(uint32_t lo, uint32_t hi, F&& pred) {
  const uint32_t lane = threadIdx.x & (WAVE - 1);
  while (lo < hi) {
    const uint32_t step = (hi - lo + WAVE - 1) / WAVE;
    const uint32_t k = lo + lane * step;
    const bool valid = k < hi;
    const uint64_t yes = __ballot(valid && pred(k));
    if (yes) {
      const uint32_t f = (uint32_t)(__ffsll((long long)yes) - 1);
      const uint32_t kf = lo + f * step;
      lo = f == 0 ? lo : kf - step + 1;  // lane f - 1's key fails
      hi = kf;
    } else {
      lo = lo + (uint32_t)(63 - __clzll((long long)__ballot(valid))) * step + 1;  // past the last key tried
    }
  }
  return lo;
}

// wave_first_key with a guess of the answer: one round over the 64 keys from guess - 32, which
// settles it when the boundary lies among them (the usual case for a guess from the closed form
// of the predicate); otherwise the search goes on over the side of that round that holds it.
template <class F>
__device__ __forceinline__ uint32_t wave_first_key_near(uint32_t lo, uint32_t hi, uint32_t guess, F&& pred) {
  if (lo >= hi) return lo;
  const uint32_t lane = threadIdx.x & (WAVE - 1);
  uint32_t g0 = guess > lo + WAVE / 2 ? guess - WAVE / 2 : lo;
  if (g0 >= hi) g0 = hi - 1;
  const uint32_t k = g0 + lane;
  const bool valid = k < hi;
  const uint64_t yes = __ballot(valid && pred(k));
  if (yes & 1ull) return wave_first_key(lo, g0, pred);  // key g0 holds: the boundary is at or below it
  if (yes) return g0 + (uint32_t)(__ffsll((long long)yes) - 1);
  const uint32_t past = g0 + (uint32_t)(64 - __clzll((long long)__ballot(valid)));  // past the last key tried
  return past >= hi ? hi : wave_first_key(past, hi, pred);
}

// Element e (a run-time index) of a vector, and its replacement: branch-free, through the two
// 64-bit halves of the vector.
template <int DT>
__device__ __forceinline__ float vec_elem_dyn(const uint4& v, int e) {
  constexpr int per_half = DT == DSV_BF16 ? 4 : 2;
  constexpr int bits = DT == DSV_BF16 ? 16 : 32;
  const uint64_t lo = ((uint64_t)v.y << 32) | v.x, hi = ((uint64_t)v.w << 32) | v.z;
  const uint64_t h = e >= per_half ? hi : lo;
  const uint32_t w = (uint32_t)(h >> (bits * (e & (per_half - 1))));
  return DT == DSV_BF16 ? __uint_as_float(w << 16) : __uint_as_float(w);
}
template <int DT>
__device__ __forceinline__ void vec_set_dyn(uint4& v, int e, float x) {
  constexpr int per_half = DT == DSV_BF16 ? 4 : 2;
  constexpr int bits = DT == DSV_BF16 ? 16 : 32;
  constexpr uint64_t ones = DT == DSV_BF16 ? 0xffffull : 0xffffffffull;
  uint64_t lo = ((uint64_t)v.y << 32) | v.x, hi = ((uint64_t)v.w << 32) | v.z;
  const bool upper = e >= per_half;
  const int sh = bits * (e & (per_half - 1));
  const uint64_t nv = (uint64_t)(DT == DSV_BF16 ? (__float_as_uint(x) >> 16) : __float_as_uint(x));
  const uint64_t h = ((upper ? hi : lo) & ~(ones << sh)) | (nv << sh);
  lo = upper ? lo : h;
  hi = upper ? h : hi;
  v = make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

// Vector vi of a 16-byte-aligned row, no bounds check (the caller knows it is inside).
// A raw buffer over [base, base + bytes): loads past the end return zeros, and each load takes
// a 32-bit lane offset plus a scalar offset (no 64-bit address arithmetic per load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at lane offset voff + scalar offset soff, streamed (non-temporal).
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  const auto t = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, (int)soff, 2);
  return make_uint4(t[0], t[1], t[2], t[3]);
}
// The same load with the default cache policy (the lines stay in the caches for a later reader).
__device__ __forceinline__ uint4 buf_load16_cached(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  const auto t = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, (int)soff, 0);
  return make_uint4(t[0], t[1], t[2], t[3]);
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)voff, (int)soff, 0);
}

__device__ __forceinline__ uint4 load_vec_raw(const char* rowp, int64_t vi) {
  const v4u_t t = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(rowp) + vi);
  return make_uint4(t.x, t.y, t.z, t.w);
}

// Replace element e of a vector by x (bf16 values are exact: the penalty rounds to bf16).
template <int DT>
__device__ __forceinline__ void vec_set(uint4& v, int e, float x) {
  uint32_t* w = reinterpret_cast<uint32_t*>(&v);
  if constexpr (DT == DSV_BF16) {
    const uint32_t b = __float_as_uint(x) >> 16;
    uint32_t& d = w[e >> 1];
    d = (e & 1) ? ((d & 0xffffu) | (b << 16)) : ((d & 0xffff0000u) | b);
  } else {
    w[e] = __float_as_uint(x);
  }
}

// Presence (additive) then repetition (multiplicative) penalty of one history token, each
// step rounded to the logits dtype as the reference's in-place tensor ops do.
// Branch-free (both the product and the quotient are formed); finite and infinite inputs.
__device__ __forceinline__ float round_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}
template <int DT>
__device__ __forceinline__ float penalize(float x, float presence, float repetition) {
  float x1 = x + (-presence);
  if constexpr (DT == DSV_BF16) x1 = round_bf16(x1);
  const float scaled = x1 * repetition;
  const float divided = x1 / repetition;
  float x2 = x1 < 0.f ? scaled : divided;
  if constexpr (DT == DSV_BF16) x2 = round_bf16(x2);
  return x2;
}

// Penalty bitmap of request b's history over ids [lo, lo + 32*words) in LDS.
__device__ __forceinline__ void build_bitmap(const dsv_verify_args& a, int b, int64_t lo, int words,
                                             uint32_t* bm) {
  for (int i = threadIdx.x; i < words; i += blockDim.x) bm[i] = 0u;
  __syncthreads();
  const int32_t* h = a.hist_ids + (int64_t)b * a.hist_len;
  const int64_t hi = lo + (int64_t)words * 32;
  for (int i = threadIdx.x; i < a.hist_len; i += blockDim.x) {
    const int64_t t = h[i];
    if (t >= lo && t < hi && t < a.vocab) {
      const int64_t o = t - lo;
      atomicOr(&bm[o >> 5], 1u << (o & 31));
    }
  }
  __syncthreads();
}
__device__ __forceinline__ bool bitmap_test(const uint32_t* bm, int64_t o) { return (bm[o >> 5] >> (o & 31)) & 1u; }

// Is token t in request b's history?  (one wave scans the history with a ballot)
__device__ __forceinline__ bool in_history_wave(const dsv_verify_args& a, int b, int64_t t) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int32_t* h = a.hist_ids + (int64_t)b * a.hist_len;
  bool hit = false;
  for (int i = lane; i < a.hist_len; i += WAVE) hit |= (int64_t)h[i] == t;
  return __ballot(hit) != 0ull;
}

// log2(e) / T: the scale of the running softmax sums exp2((x - m) * log2(e) / T).
__device__ __forceinline__ float log2e_over(float T) { return 1.44269504088896340736f * __builtin_amdgcn_rcpf(T); }

// p(x) = fp32(exp(fp32(x / T) - m_f) * invZ): the unfiltered softmax probability.
__device__ __forceinline__ float prob_of(float x, float T, float m_f, float invZ) {
  const float xf = x / T;
  return expf(xf - m_f) * invZ;
}

// P at one value of a dense row (unfiltered, or a nucleus row's kept value): p, renormalised
// over the kept mass when the row is filtered.
__device__ __forceinline__ double dense_P(const RowSum& rs, float T, float x) {
  const float p = prob_of(x, T, rs.m_f, rs.invZ);
  return (rs.mode == M_HIST || rs.norm) ? (double)(p / rs.S_f) : (double)p;
}

// ---------------------------------------------------------------------------------------
// Candidate selection on packed (key, ~id) values (distinct, larger = better)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t pack(uint32_t key, int64_t j) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j);
}
__device__ __forceinline__ int32_t unpack_id(uint64_t p) { return (int32_t)(0xFFFFFFFFu - (uint32_t)p); }
__device__ __forceinline__ uint32_t unpack_key(uint64_t p) { return (uint32_t)(p >> 32); }

// The k-th largest of buf[0..n) (1 <= k <= n, values distinct), by the calling wave with an
// 8-bit-digit radix select over an LDS histogram.
__device__ inline uint64_t wave_kth_largest(const uint64_t* buf, int n, int k, uint32_t* hist, int top_shift) {
  const int lane = threadIdx.x & (WAVE - 1);
  uint64_t prefix = 0, mask = 0;
  for (int shift = top_shift; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += WAVE) hist[i] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int base = 0; base < n; base += WAVE) {
      const int i = base + lane;
      const uint64_t v = i < n ? buf[i] : 0ull;
      const bool m = i < n && (v & mask) == prefix;
      const uint32_t d = (uint32_t)(v >> shift) & 255u;
      const uint64_t bal = __ballot(m);
      if (bal == 0ull) continue;
      const int first = __ffsll((long long)bal) - 1;
      const uint32_t d0 = __shfl(d, first, WAVE);
      const uint64_t same = __ballot(m && d == d0);
      if (same == bal) {
        if (lane == first) atomicAdd(&hist[d0], (uint32_t)__popcll(bal));
      } else if (m) {
        atomicAdd(&hist[d], 1u);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint32_t c[4];
    uint32_t tot = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = hist[255 - 4 * lane - q];
      tot += c[q];
    }
    const uint32_t incl = wave_incl_scan(tot);
    const uint32_t excl = incl - tot;
    int digit = -1, knew = 0;
    if ((uint32_t)k > excl && (uint32_t)k <= incl) {
      uint32_t run = excl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (digit < 0) {
          if (run + c[q] >= (uint32_t)k) {
            digit = 255 - 4 * lane - q;
            knew = k - (int)run;
          } else {
            run += c[q];
          }
        }
      }
    }
    const uint64_t who = __ballot(digit >= 0);
    const int src = who ? (__ffsll((long long)who) - 1) : 0;
    digit = __shfl(digit, src, WAVE);
    knew = __shfl(knew, src, WAVE);
    if (digit < 0) break;
    k = knew;
    prefix |= (uint64_t)digit << shift;
    mask |= 0xFFull << shift;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  return prefix;
}

// Keep the k largest of buf[0..n) in buf[0..min(k,n)), sorted descending.  Block-wide call;
// `top` holds >= min(k, n) entries and `cnt` is an LDS int.
template <int TOP_SHIFT>
__device__ int select_top(uint64_t* buf, int n, int k, uint64_t* top, uint32_t* hist, uint64_t* sh,
                          int* cnt) {
  const int kk = k < n ? k : n;
  if (kk <= 0) return 0;
  if (threadIdx.x < WAVE) {
    const uint64_t t = wave_kth_largest(buf, n, kk, hist, TOP_SHIFT);
    if (threadIdx.x == 0) {
      sh[0] = t;
      *cnt = 0;
    }
  }
  __syncthreads();
  const uint64_t tk = sh[0];
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const uint64_t v = buf[i];
    if (v >= tk) top[atomicAdd(cnt, 1)] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kk; i += blockDim.x) {
    const uint64_t mine = top[i];
    int rank = 0;
    for (int j = 0; j < kk; ++j) rank += top[j] > mine;
    buf[rank] = mine;
  }
  __syncthreads();
  return kk;
}

// pytorch backend: zero when fp32(fp32(S_j) - p_j) > top_p, S_j the prefix sum including p_j
// (double, as CPU cumsum accumulates); flashinfer joint: mass strictly ahead > top_p.
__device__ __forceinline__ bool topp_fails(int backend, double S_before, float p, float top_p) {
  if (backend == DSV_BACKEND_PYTORCH) {
    const float Sj = (float)(S_before + (double)p);
    return (Sj - p) > top_p;
  }
  return S_before > (double)top_p;
}

__device__ __forceinline__ float clamp01(float q) { return (q >= 0.f && q <= 1.f) ? q : 0.f; }

// Whether a support-list (top-k) row of the verify step needs its softmax normaliser Z: only a
// top-p test on the unrenormalised probabilities reads it.  Top-k and min-p compare p up to a
// common factor, the flashinfer min-p branch renormalises over the top-k before its top-p test,
// and with top_p >= 1 the test keeps every value (up to the float32 rounding of its running
// sum).  The target-distribution entry reports p / Z and always needs it.
__device__ __forceinline__ bool list_needs_z(const dsv_verify_args& a, float top_p) {
  if (!a.candidates) return true;
  if (a.backend == DSV_BACKEND_FLASHINFER && a.need_min_p) return false;
  return top_p < 1.f;
}

// The first cut tie of a key held by cnt values of probability p each, with mass sb and cb values
// ahead of it in (value desc, id asc) order: the top-k rank, the min-p floor and the top-p test
// are each monotone along that order.  Returns cnt when none of the ties is cut.
__device__ __forceinline__ int64_t cut_index(int backend, int64_t cnt, float p, double sb, int64_t cb, int topk,
                                             float min_p, float thr_minp, float top_p) {
  int64_t fail = cnt;
  if (min_p > 0.f && p < thr_minp) fail = 0;
  if (cb >= (int64_t)topk)
    fail = 0;
  else if (cb + cnt > (int64_t)topk)
    fail = fail < (int64_t)topk - cb ? fail : (int64_t)topk - cb;
  if (fail > 0 && topp_fails(backend, sb + (double)(cnt - 1) * (double)p, p, top_p)) {
    int64_t l0 = 0, l1 = cnt - 1;  // smallest failing tie
    while (l0 < l1) {
      const int64_t mid = (l0 + l1) >> 1;
      if (topp_fails(backend, sb + (double)mid * (double)p, p, top_p))
        l1 = mid;
      else
        l0 = mid + 1;
    }
    fail = fail < l0 ? fail : l0;
  }
  return fail;
}

// Append the lanes' values with h set to buf (slots from an LDS counter; values past cap are
// counted but dropped).
__device__ __forceinline__ void wave_append(bool h, uint64_t v, uint64_t* buf, int cap, int32_t* cnt) {
  const uint64_t bal = __ballot(h);
  if (bal == 0ull) return;
  const int lane = threadIdx.x & (WAVE - 1);
  const int first = __ffsll((long long)bal) - 1;
  int base = 0;
  if (lane == first) base = atomicAdd(cnt, __popcll(bal));
  base = __shfl(base, first, WAVE);
  if (h) {
    const int slot = base + __popcll(bal & ((1ull << lane) - 1ull));
    if (slot < cap) buf[slot] = v;
  }
}

// Chain-rejection test of step s of request b (sampling/sparse/accept.py:249-283): the draft
// token is accepted iff q > 0 and q <= 1 and u * q < p, where q sums, in lane order, the
// sparse-q lanes holding the token and p is the target probability of the token.  Called by
// one full wave; every lane returns the decision.
__device__ __forceinline__ int32_t step_accept_wave(const dsv_verify_args& a, int b, int s, int64_t tok, float p) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int64_t qi = ((int64_t)b * (a.T - 1) + s) * a.K;
  const bool hit = lane < a.K && load_index(a.q_ids, a.q_ids_i64, qi + lane) == tok;
  uint64_t bal = __ballot(hit);
  float q = 0.f;
  while (bal) {
    const int l = __ffsll((long long)bal) - 1;
    bal &= bal - 1ull;
    q += a.q_values[qi + l];
  }
  const float coin = a.uniforms[(int64_t)b * (a.T - 1) + s];
  return (q > 0.f && q <= 1.f && coin * q < p) ? 1 : 0;
}

// Block-wide inclusive prefix of doubles in thread order, as tiles: thread t gets [lo, hi)
// with hi(t) == lo(t + 1) bit for bit, so that exactly one thread holds any point below the
// total.  `scratch` holds one double per wave; returns the total (== hi of the last thread).
template <int NW>
__device__ __forceinline__ double block_tiles(double v, double* scratch, double& lo, double& hi) {
  const int lane = threadIdx.x & (WAVE - 1), wid = threadIdx.x / WAVE;
  constexpr int nw = NW;
  const double incl = wave_incl_scan(v);
  __syncthreads();
  if (lane == WAVE - 1) scratch[wid] = incl;
  __syncthreads();
  double base = 0.0, tot = 0.0;
  for (int i = 0; i < nw; ++i) {
    if (i == wid) base = tot;
    tot += scratch[i];
  }
  hi = base + incl;
  lo = wave_prev(hi, base);
  (void)lane;
  return tot;
}

// The same over the lanes of one wave (values of lanes >= n count as zero).
__device__ __forceinline__ double wave_tiles(double v, double& lo, double& hi) {
  hi = wave_incl_scan(v);
  lo = wave_prev(hi, 0.0);
  return readlane<WAVE - 1>(hi);
}

}  // namespace dsv
