// Sampled draft verification for gfx950: target distribution, chain rejection with sparse q,
// residual resample, accepted-prefix compaction and KV-slot gather.
//
// Three launches per verify step (all on the caller's stream, no host synchronisation):
//   k_rows      one 1024-thread workgroup per verified target row.  One read of the row
//               computes everything the rejection walk needs from it:
//                 GREEDY  rows of top_k <= 1 requests: first argmax (one-hot target)
//                 LIST    filtered rows with top_k <= 64: running softmax sum + exact top-k
//                         candidate selection -> the filtered target support as (id, P) pairs
//                 UNF     unfiltered rows: running softmax sum (P = softmax)
//                 HIST    filtered rows with large top_k (nucleus): an LDS histogram of the
//                         65536 bf16 values; Z, the top-k/top-p/min-p cut (key + tie count)
//                         and the normaliser all follow from value counts
//               and P at the row's draft token.
//   k_chunks    (request, chunk) workgroups: the rejection walk, then -- only when the bonus
//               row has a dense support (UNF / HIST) -- per-chunk residual masses of that row.
//   k_finalize  one workgroup per request: residual CDF -> bonus token (from the support
//               list, or by locating the chunk and rescanning it), then the outputs.
//
// Semantics follow runtime/worker.py:440-508 (target P, pytorch backend), sampling/rejection.py
// :36-98 and sampling/sparse/accept.py:239-307 (chain rejection); see the oracle for the
// CPU restatement.
#include <float.h>
#include <limits.h>
#include <string.h>

#include "dsv_common.h"

namespace dsv {

enum RowMode { M_SKIP = 0, M_GREEDY = 1, M_LIST = 2, M_UNF = 3, M_HIST = 4 };

struct RowSum {
  int32_t mode;
  int32_t argmax;   // first maximal id of the adjusted row
  uint32_t kmax;    // key of the maximum
  uint32_t vcut;    // HIST: kept iff key > vcut or (key == vcut and tie rank < ktie)
  int32_t ktie;
  int32_t nlist;    // LIST/GREEDY: number of support entries
  float m_f;        // fp32(max / T)
  float invZ;       // fp32(1 / Z)
  float S_f;        // normaliser of the filtered row (1 when unfiltered)
  float p_draft;    // P at this row's draft token
  int32_t flags;
  int32_t pad;
  double Z;
  double S_kept;
};
static_assert(sizeof(RowSum) == 64, "RowSum layout");

struct ListEntry {
  int32_t id;
  float P;
};
struct ReqState {
  int32_t a, all, rstar, mode;
};
struct ChunkSum {
  double mass;   // residual-free mass of kept ids with key > vcut (HIST) / all ids (UNF)
  int32_t ties;  // ids with key == vcut (HIST)
  int32_t pad;
};

constexpr int ROW_THREADS = 1024;
constexpr int LIST_U = 2;                        // vectors per thread per block in LIST mode
constexpr int LIST_BLOCK = ROW_THREADS * 8 * LIST_U;
constexpr int LIST_CAP = LIST_BLOCK + 256;       // candidate buffer entries
constexpr int HIST_WORDS = 32768;                // 65536 16-bit counters
constexpr int NCH = 32;                          // chunks per bonus row
constexpr int CHUNK_THREADS = 256;
constexpr int QMAX = 64;                         // largest supported sparse-q width K
constexpr int FLAG_HIST_OVERFLOW = 1;

struct KParams {
  dsv_verify_args a;
  RowSum* rowsum;
  ListEntry* lists;
  ReqState* req;
  ChunkSum* chunks;
  int32_t* qrank;      // [bs, QMAX]: tie rank of each q lane id inside its chunk
  int64_t chunk;       // elements per chunk (multiple of 8)
  int32_t aligned;     // logits rows are 16-byte aligned
  int32_t bitmap_words;
  int32_t force_greedy;
  int32_t pad;
};

// ---------------------------------------------------------------------------------------
// Element access
// ---------------------------------------------------------------------------------------
template <int DT>
struct Raw;
template <>
struct Raw<DSV_BF16> {
  uint4 v;
};
template <>
struct Raw<DSV_F32> {
  uint4 v[2];
};

template <int DT>
__device__ __forceinline__ void load_raw(Raw<DT>& r, const char* rowp, int64_t vi, int64_t V,
                                         bool aligned) {
  const int64_t j0 = vi * 8;
  if constexpr (DT == DSV_BF16) {
    if (aligned && j0 + 8 <= V) {
      r.v = *reinterpret_cast<const uint4*>(rowp + j0 * 2);
    } else {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(rowp);
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = (j0 + e < V) ? p[j0 + e] : 0xFF80u;
      r.v = make_uint4(w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16),
                       w[6] | (w[7] << 16));
    }
  } else {
    if (aligned && j0 + 8 <= V) {
      const uint4* q = reinterpret_cast<const uint4*>(rowp + j0 * 4);
      r.v[0] = q[0];
      r.v[1] = q[1];
    } else {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(rowp);
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = (j0 + e < V) ? p[j0 + e] : 0xFF800000u;
      r.v[0] = make_uint4(w[0], w[1], w[2], w[3]);
      r.v[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
  }
}

template <int DT>
__device__ __forceinline__ void decode(const Raw<DT>& r, float x[8]) {
  if constexpr (DT == DSV_BF16) {
    const uint32_t w[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const uint32_t w[8] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w,
                           r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = __uint_as_float(w[i]);
  }
}

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

// Presence (additive) then repetition (multiplicative) penalty of one history token, each
// step rounded to the logits dtype as the reference's in-place tensor ops do.
template <int DT>
__device__ __forceinline__ float penalize(float x, float presence, float repetition) {
  float x1 = x + (-presence);
  if constexpr (DT == DSV_BF16) x1 = bf16_bits_to_f32(f32_to_bf16_bits(x1));
  float x2 = x1 < 0.f ? x1 * repetition : x1 / repetition;
  if constexpr (DT == DSV_BF16) x2 = bf16_bits_to_f32(f32_to_bf16_bits(x2));
  return x2;
}

template <int DT>
__device__ __forceinline__ float load_elem(const char* rowp, int64_t j) {
  if constexpr (DT == DSV_BF16)
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(rowp)[j]);
  else
    return reinterpret_cast<const float*>(rowp)[j];
}

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

// Verified rows of request b: verify_lens[b] clamped to [1, T] so that a bad length can never
// index past the candidates / q / uniforms of its request.
__device__ __forceinline__ int req_cap(const dsv_verify_args& a, int b) {
  int cap = a.verify_lens ? a.verify_lens[b] : a.T;
  return cap < 1 ? 1 : (cap > a.T ? a.T : cap);
}

// Row r -> (request b, position s); false when r is not a verified row.
__device__ __forceinline__ bool row_request(const dsv_verify_args& a, int64_t r, int& b, int& s) {
  if (a.row_offsets == nullptr) {
    b = (int)(r / a.T);
    s = (int)(r - (int64_t)b * a.T);
  } else {
    int lo = 0, hi = a.bs - 1;
    if (load_index(a.row_offsets, a.row_offsets_i64, 0) > r) return false;
    while (lo < hi) {  // largest b with offset[b] <= r
      int mid = (lo + hi + 1) >> 1;
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

__device__ __forceinline__ int row_mode(const dsv_verify_args& a, int b, int force_greedy) {
  if (force_greedy) return M_GREEDY;
  const int k = a.top_ks[b];
  if (a.any_greedy && k <= 1) return M_GREEDY;
  if (!a.filter) return M_UNF;
  return k <= DSV_LIST_K ? M_LIST : M_HIST;
}

// Penalty bitmap of request b's history over [lo, lo + 32*words) in LDS.
__device__ void build_bitmap(const dsv_verify_args& a, int b, int64_t lo, int words, uint32_t* bm) {
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

__device__ __forceinline__ bool bitmap_test(const uint32_t* bm, int64_t o) {
  return (bm[o >> 5] >> (o & 31)) & 1u;
}

// p(x) = fp32(exp(fp32(x / T) - m_f) * invZ): the unfiltered softmax probability.
__device__ __forceinline__ float prob_of(float x, float T, float m_f, float invZ) {
  const float xf = x / T;
  return expf(xf - m_f) * invZ;
}

// ---------------------------------------------------------------------------------------
// Candidate selection: K-th largest of distinct 64-bit packed (key, ~id) values in LDS,
// by one wave with an 8-bit-digit radix select.
// ---------------------------------------------------------------------------------------
__device__ uint64_t wave_kth_largest(const uint64_t* buf, int n, int k, uint32_t* hist, int top_shift) {
  const int lane = threadIdx.x & (WAVE - 1);
  uint64_t prefix = 0, mask = 0;
  for (int shift = top_shift; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += WAVE) hist[i] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int base = 0; base < n; base += WAVE) {
      const int i = base + lane;
      uint64_t v = i < n ? buf[i] : 0ull;
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
    // lane l owns digits 255-4l .. 252-4l (descending)
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
    if (digit < 0) break;  // k > n: not reached by callers
    k = knew;
    prefix |= (uint64_t)digit << shift;
    mask |= 0xFFull << shift;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  return prefix;
}

// Keep the k largest of buf[0..n) (distinct values), compacting them into buf[0..k) in
// descending order.  All threads of the block call it.  Returns k' = min(k, n).
template <int TOP_SHIFT>
__device__ int select_top(uint64_t* buf, int n, int k, uint64_t* top, uint32_t* hist,
                          uint64_t* sh) {
  const int kk = k < n ? k : n;
  if (kk <= 0) return 0;
  if (threadIdx.x < WAVE) {
    const uint64_t t = wave_kth_largest(buf, n, kk, hist, TOP_SHIFT);
    if (threadIdx.x == 0) sh[0] = t;
  }
  __syncthreads();
  const uint64_t tk = sh[0];
  // every kept value has rank < kk among the kept: write it at its rank
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const uint64_t v = buf[i];
    if (v >= tk) {
      int rank = 0;
      for (int j = 0; j < n; ++j) rank += buf[j] > v;
      top[rank] = v;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kk; i += blockDim.x) buf[i] = top[i];
  __syncthreads();
  return kk;
}

// Same, but the rank search only scans the survivors (cheap when n is large).
template <int TOP_SHIFT>
__device__ int select_top_fast(uint64_t* buf, int n, int k, uint64_t* top, uint32_t* hist,
                               uint64_t* sh, int* cnt) {
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
  // sort the kk survivors (descending) by rank
  uint64_t mine = 0;
  int myrank = -1;
  if ((int)threadIdx.x < kk) {
    mine = top[threadIdx.x];
    int rank = 0;
    for (int j = 0; j < kk; ++j) rank += top[j] > mine;
    myrank = rank;
  }
  __syncthreads();
  if (myrank >= 0) buf[myrank] = mine;
  __syncthreads();
  return kk;
}

__device__ __forceinline__ uint64_t pack(uint32_t key, int64_t j) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j);
}
__device__ __forceinline__ int32_t unpack_id(uint64_t p) { return (int32_t)(0xFFFFFFFFu - (uint32_t)p); }
__device__ __forceinline__ uint32_t unpack_key(uint64_t p) { return (uint32_t)(p >> 32); }

// ---------------------------------------------------------------------------------------
// Target-filter tests on the sorted prefix (runtime/worker.py:52-67 pytorch backend;
// S2 joint semantics for flashinfer).
// ---------------------------------------------------------------------------------------
// pytorch: zero when fp32(fp32(S_j) - p_j) > top_p, S_j = prefix sum (double, CPU cumsum)
__device__ __forceinline__ bool topp_fails(int backend, double S_before, float p, float top_p) {
  if (backend == DSV_BACKEND_PYTORCH) {
    const float Sj = (float)(S_before + (double)p);
    return (Sj - p) > top_p;
  }
  return S_before > (double)top_p;  // mass ahead > top_p
}

// ---------------------------------------------------------------------------------------
// k_rows
// ---------------------------------------------------------------------------------------
struct RowShared {
  double d[16];
  uint64_t u[16];
  float f[16];
  int32_t i[32];
  uint32_t hist256[256];
  uint64_t top[DSV_LIST_K];
  uint64_t misc[4];
  float xtok;
  uint32_t ktok;
  int32_t cnt;
  int32_t cnt2;
  uint64_t thr;
};

template <int DT, int MODE>
__device__ void row_work(const KParams& P, int64_t r, int b, int s, RowShared& sh,
                         unsigned char* dyn) {
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const size_t esize = DT == DSV_BF16 ? 2 : 4;
  const char* rowp = reinterpret_cast<const char*>(a.logits) + (size_t)r * (size_t)a.row_stride * esize;
  const bool aligned = P.aligned != 0;
  const int cap = req_cap(a, b);
  const float T = MODE == M_GREEDY ? 1.f : a.temperatures[b];
  const int topk = MODE == M_GREEDY ? 1 : a.top_ks[b];

  // LDS regions: [0, 133120) candidates or histogram; then the penalty bitmap.
  uint64_t* cbuf = reinterpret_cast<uint64_t*>(dyn);
  uint32_t* hist = reinterpret_cast<uint32_t*>(dyn);
  uint32_t* bm = reinterpret_cast<uint32_t*>(dyn + (size_t)LIST_CAP * 8);
  const bool pen = a.hist_ids != nullptr && P.bitmap_words > 0;
  float pres = 0.f, rep = 1.f;
  if (pen) {
    pres = a.presence ? a.presence[b] : 0.f;
    rep = a.repetition ? a.repetition[b] : 1.f;
    build_bitmap(a, b, 0, P.bitmap_words, bm);
  }
  if constexpr (MODE == M_HIST) {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
    for (int i = tid; i < HIST_WORDS / 4; i += ROW_THREADS) h4[i] = make_uint4(0, 0, 0, 0);
  }
  // the draft token checked against this row
  const int64_t tok = (s < cap - 1 && s + 1 < a.T) ? a.candidates[(int64_t)b * a.T + s + 1] : -1;
  if (tid == 0) {
    float xt = -INFINITY;
    if (tok >= 0 && tok < V) {
      xt = load_elem<DT>(rowp, tok);
      if (pen && bitmap_test(bm, tok)) xt = penalize<DT>(xt, pres, rep);
    }
    sh.xtok = xt;
    sh.ktok = key_of<DT>(xt);
    sh.cnt = 0;
    sh.thr = 0ull;
  }
  __syncthreads();
  const uint32_t ktok = sh.ktok;

  const float c2 = 1.44269504088896340736f / T;  // log2(e) / T for the running sums
  uint64_t best = 0ull;                          // packed (key, ~id): max key, lowest id
  float m_t = -INFINITY, s_t = 0.f;
  uint32_t tie_before = 0, nfin = 0;
  constexpr int U = MODE == M_LIST ? LIST_U : 4;
  const int64_t NVt = (V + 7) / 8;
  const int lane = tid & (WAVE - 1), wid = tid / WAVE;

  for (int64_t v0 = 0; v0 < NVt; v0 += (int64_t)ROW_THREADS * U) {
    Raw<DT> raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + (int64_t)u * ROW_THREADS + tid;
      if (vi < NVt) load_raw<DT>(raw[u], rowp, vi, V, aligned);
    }
    uint32_t keys[U][8];
    float xs[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + (int64_t)u * ROW_THREADS + tid;
      if (vi >= NVt) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          keys[u][e] = 0u;
          xs[u][e] = -INFINITY;
        }
        continue;
      }
      float x[8];
      decode<DT>(raw[u], x);
      if (pen) {
        const uint32_t byte = (bm[vi >> 2] >> ((vi & 3) * 8)) & 0xFFu;
        if (byte) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if ((byte >> e) & 1u) x[e] = penalize<DT>(x[e], pres, rep);
        }
      }
      float vmax = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t j = vi * 8 + e;
        const bool valid = j < V;
        const uint32_t k = key_of<DT>(x[e]);
        keys[u][e] = k;
        xs[u][e] = valid ? x[e] : -INFINITY;
        const uint64_t pk = valid ? pack(k, j) : 0ull;
        best = pk > best ? pk : best;
        vmax = fmaxf(vmax, xs[u][e]);
        if constexpr (MODE == M_HIST) {
          if (valid && k != NEG_INF_BF16_KEY) {
            atomicAdd(&hist[k >> 1], 1u << ((k & 1u) * 16u));
            ++nfin;
            tie_before += (k == ktok && j < tok) ? 1u : 0u;
          }
        }
      }
      if constexpr (MODE == M_UNF || MODE == M_LIST) {
        if (vmax > m_t) {
          s_t *= __builtin_amdgcn_exp2f((m_t - vmax) * c2);
          m_t = vmax;
        }
        if (m_t > -INFINITY) {
#pragma unroll
          for (int e = 0; e < 8; ++e) s_t += __builtin_amdgcn_exp2f((xs[u][e] - m_t) * c2);
        }
      }
    }
    if constexpr (MODE == M_LIST) {
      const int K = topk < 1 ? 1 : topk;
      if (v0 == 0) {
        // admission bound from this block: min over waves of each wave's ceil(K/16)-th
        // largest thread maximum (>= K distinct elements lie at or above it)
        uint64_t tm = 0ull;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int64_t j = (v0 + (int64_t)u * ROW_THREADS + tid) * 8 + e;
            const uint64_t pk = j < V ? pack(keys[u][e], j) : 0ull;
            tm = pk > tm ? pk : tm;
          }
        const int J = (K + 15) / 16;
        uint64_t w = 0ull;
        for (int i = 0; i < J; ++i) {
          w = wave_max_u64(tm);
          if (tm == w) tm = 0ull;
        }
        if (lane == 0) sh.u[wid] = w;
        __syncthreads();
        if (tid == 0) {
          uint64_t t0 = ~0ull;
          for (int i = 0; i < ROW_THREADS / WAVE; ++i) t0 = sh.u[i] < t0 ? sh.u[i] : t0;
          sh.thr = t0;
        }
        __syncthreads();
      }
      const uint64_t thr = sh.thr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t hits = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t j = (v0 + (int64_t)u * ROW_THREADS + tid) * 8 + e;
          hits |= (j < V && pack(keys[u][e], j) >= thr) ? (1u << e) : 0u;
        }
        if (__ballot(hits != 0u) == 0ull) continue;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool h = (hits >> e) & 1u;
          const uint64_t bal = __ballot(h);
          if (bal == 0ull) continue;
          const int first = __ffsll((long long)bal) - 1;
          int base = 0;
          if (lane == first) base = atomicAdd(&sh.cnt, __popcll(bal));
          base = __shfl(base, first, WAVE);
          if (h) {
            const int slot = base + __popcll(bal & ((1ull << lane) - 1ull));
            const int64_t j = (v0 + (int64_t)u * ROW_THREADS + tid) * 8 + e;
            if (slot < LIST_CAP) cbuf[slot] = pack(keys[u][e], j);
          }
        }
      }
      __syncthreads();
      int n = sh.cnt;
      if (n > LIST_CAP) n = LIST_CAP;  // not reachable: compaction keeps room for a block
      if (v0 == 0 || n > LIST_CAP - LIST_BLOCK) {
        const int kk = select_top_fast<DT == DSV_BF16 ? 40 : 56>(cbuf, n, K, sh.top, sh.hist256,
                                                                 sh.misc, &sh.cnt2);
        if (tid == 0) {
          sh.cnt = kk;
          if (kk == K) sh.thr = cbuf[K - 1] + 1ull;  // later ids must beat the K-th largest
        }
        __syncthreads();
      }
    }
  }

  // ---- block results ----------------------------------------------------------------
  const uint64_t gbest = block_max_u64(best, sh.u);
  const uint32_t kmax = unpack_key(gbest);
  const int32_t argmax = gbest ? unpack_id(gbest) : 0;
  RowSum rs;
  rs.mode = MODE;
  rs.argmax = argmax;
  rs.kmax = kmax;
  rs.vcut = 0u;
  rs.ktie = INT_MAX;
  rs.nlist = 0;
  rs.flags = 0;
  rs.pad = 0;
  rs.S_f = 1.f;
  rs.S_kept = 1.0;
  rs.Z = 1.0;
  const float M = value_of_key<DT>(kmax);
  const float m_f = M / T;
  rs.m_f = m_f;
  rs.invZ = 1.f;
  rs.p_draft = 0.f;
  ListEntry* list = P.lists + r * DSV_LIST_K;

  if constexpr (MODE == M_GREEDY) {
    rs.nlist = 1;
    rs.p_draft = (tok == argmax) ? 1.f : 0.f;
    if (tid == 0) list[0] = ListEntry{argmax, 1.f};
  }

  if constexpr (MODE == M_UNF || MODE == M_LIST) {
    double zt = 0.0;
    if (m_t > -INFINITY) zt = (double)s_t * (double)__builtin_amdgcn_exp2f((m_t - M) * c2);
    const double Z = block_sum(zt, sh.d);
    rs.Z = Z;
    rs.invZ = (float)(1.0 / Z);
    if constexpr (MODE == M_UNF) {
      rs.p_draft = (tok >= 0 && tok < V) ? prob_of(sh.xtok, T, m_f, rs.invZ) : 0.f;
    }
  }

  if constexpr (MODE == M_LIST) {
    // final exact top-K, already sorted descending in cbuf[0..kk)
    const int K = topk < 1 ? 1 : topk;
    int n = sh.cnt;
    if (n > LIST_CAP) n = LIST_CAP;
    __syncthreads();
    const int kk = select_top_fast<DT == DSV_BF16 ? 40 : 56>(cbuf, n, K, sh.top, sh.hist256, sh.misc,
                                                             &sh.cnt2);
    if (tid == 0) {
      // filter tests on the sorted prefix, then normalise the kept mass
      const float top_p = a.top_ps[b];
      const float min_p = a.min_ps ? a.min_ps[b] : 0.f;
      float pv[DSV_LIST_K];
      bool keep[DSV_LIST_K];
      double S = 0.0;
      float p0 = 0.f;
      for (int j = 0; j < kk; ++j) {
        const float x = value_of_key<DT>(unpack_key(cbuf[j]));
        const float p = prob_of(x, T, m_f, rs.invZ);
        pv[j] = p;
        if (j == 0) p0 = p;
        bool k_ok = j < topk;
        bool p_ok = !topp_fails(a.backend, S, p, top_p);
        S += (double)p;
        keep[j] = k_ok && p_ok;
      }
      if (a.need_min_p) {
        if (a.backend == DSV_BACKEND_FLASHINFER) {
          // sequential branch: renormalise over top-k, top-p on that mass, then min-p
          double Sk = 0.0;
          for (int j = 0; j < kk; ++j) Sk += (double)pv[j];
          double ahead = 0.0;
          for (int j = 0; j < kk; ++j) {
            const double w = (double)pv[j] / Sk;
            keep[j] = j < topk && ahead <= (double)top_p;
            ahead += w;
          }
        }
        const float thr = p0 * min_p;
        for (int j = 0; j < kk; ++j)
          if (pv[j] < thr) keep[j] = false;
      }
      double Sk = 0.0;
      for (int j = 0; j < kk; ++j)
        if (keep[j]) Sk += (double)pv[j];
      const float S_f = (float)Sk;
      rs.S_kept = Sk;
      rs.S_f = S_f;
      // kept entries sorted by id (insertion sort, kk <= 64)
      int nk = 0;
      ListEntry tmp[DSV_LIST_K];
      for (int j = 0; j < kk; ++j) {
        if (!keep[j]) continue;
        const int32_t id = unpack_id(cbuf[j]);
        const float Pj = pv[j] / S_f;
        if (id == tok) rs.p_draft = Pj;
        int pos = nk++;
        while (pos > 0 && tmp[pos - 1].id > id) {
          tmp[pos] = tmp[pos - 1];
          --pos;
        }
        tmp[pos] = ListEntry{id, Pj};
      }
      for (int j = 0; j < nk; ++j) list[j] = tmp[j];
      rs.nlist = nk;
    }
  }

  if constexpr (MODE == M_HIST) {
    __syncthreads();
    const uint32_t nfin_all = (uint32_t)block_sum((double)nfin, sh.d);
    const uint32_t tie_tok = (uint32_t)block_sum((double)tie_before, sh.d);
    // thread t owns keys [65535 - 64t - 63, 65535 - 64t], words [32767-32t-31, 32767-32t]
    const int w_hi = HIST_WORDS - 1 - 32 * tid;
    double zt = 0.0;
    double ct = 0.0;
    for (int w = w_hi; w > w_hi - 32; --w) {
      const uint32_t h = hist[w];
      if (!h) continue;
#pragma unroll
      for (int half = 1; half >= 0; --half) {
        const uint32_t c = (h >> (16 * half)) & 0xFFFFu;
        if (!c) continue;
        const uint32_t k = 2u * (uint32_t)w + (uint32_t)half;
        const float e = expf(value_of_key<DT>(k) / T - m_f);
        zt += (double)c * (double)e;
        ct += (double)c;
      }
    }
    const double Z = block_sum(zt, sh.d);
    const double counted = block_sum(ct, sh.d);
    if (counted != (double)nfin_all) rs.flags |= FLAG_HIST_OVERFLOW;
    const float invZ = (float)(1.0 / Z);
    rs.Z = Z;
    rs.invZ = invZ;
    // masses with p(k) = fp32(e(k) * invZ), then the descending prefix over threads
    double mt = 0.0;
    for (int w = w_hi; w > w_hi - 32; --w) {
      const uint32_t h = hist[w];
      if (!h) continue;
#pragma unroll
      for (int half = 1; half >= 0; --half) {
        const uint32_t c = (h >> (16 * half)) & 0xFFFFu;
        if (!c) continue;
        const uint32_t k = 2u * (uint32_t)w + (uint32_t)half;
        const float p = prob_of(value_of_key<DT>(k), T, m_f, invZ);
        mt += (double)c * (double)p;
      }
    }
    double m_total = 0.0, c_total = 0.0;
    const double sb0 = block_excl_scan(mt, sh.d, &m_total);
    const double cb0 = block_excl_scan(ct, sh.d, &c_total);
    const float top_p = a.top_ps[b];
    const float min_p = a.min_ps ? a.min_ps[b] : 0.f;
    const float p_max = prob_of(M, T, m_f, invZ);
    const float thr_minp = p_max * min_p;
    // walk this thread's keys (descending) for the first failing token
    double sb = sb0, cb = cb0;
    uint64_t found = ~0ull;  // (tid << 32) | ...: earliest thread wins
    uint32_t f_key = 0;
    int32_t f_tie = 0;
    double f_S = 0.0;
    for (int w = w_hi; w > w_hi - 32 && found == ~0ull; --w) {
      const uint32_t h = hist[w];
      if (!h) continue;
      for (int half = 1; half >= 0 && found == ~0ull; --half) {
        const uint32_t c = (h >> (16 * half)) & 0xFFFFu;
        if (!c) continue;
        const uint32_t k = 2u * (uint32_t)w + (uint32_t)half;
        const float p = prob_of(value_of_key<DT>(k), T, m_f, invZ);
        int64_t fail = c;
        if (a.need_min_p && p < thr_minp) fail = 0;
        if (cb >= (double)topk)
          fail = 0;
        else if (cb + c > (double)topk)
          fail = fail < (int64_t)(topk - (int64_t)cb) ? fail : (int64_t)(topk - (int64_t)cb);
        if (fail > 0 && topp_fails(a.backend, sb + (double)(c - 1) * (double)p, p, top_p)) {
          // smallest i with a failing top-p test (monotone in i)
          int64_t lo = 0, hi = c - 1;
          while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (topp_fails(a.backend, sb + (double)mid * (double)p, p, top_p))
              hi = mid;
            else
              lo = mid + 1;
          }
          fail = fail < lo ? fail : lo;
        }
        if (fail < (int64_t)c) {
          found = ((uint64_t)tid << 32);
          f_key = k;
          f_tie = (int32_t)fail;
          f_S = sb + (double)fail * (double)p;
        } else {
          sb += (double)c * (double)p;
          cb += (double)c;
        }
      }
    }
    const uint64_t win = block_min_u64(found, sh.u);
    if (win == ~0ull) {
      if (tid == 0) {
        rs.vcut = 0u;
        rs.ktie = INT_MAX;
        rs.S_kept = m_total;
        sh.misc[0] = 0ull;
      }
    } else if ((uint64_t)tid << 32 == win) {
      rs.vcut = f_key;
      rs.ktie = f_tie;
      rs.S_kept = f_S;
      sh.misc[0] = ((uint64_t)f_key << 32) | (uint32_t)f_tie;
      sh.d[0] = f_S;
    }
    __syncthreads();
    if (tid == 0 && win != ~0ull) {
      rs.vcut = (uint32_t)(sh.misc[0] >> 32);
      rs.ktie = (int32_t)(uint32_t)sh.misc[0];
      rs.S_kept = sh.d[0];
    }
    if (tid == 0) {
      rs.S_f = (float)rs.S_kept;
      const bool kept = ktok > rs.vcut || (ktok == rs.vcut && (int64_t)tie_tok < (int64_t)rs.ktie);
      rs.p_draft = (tok >= 0 && tok < V && kept) ? prob_of(sh.xtok, T, m_f, invZ) / rs.S_f : 0.f;
    }
  }
  if (tid == 0) P.rowsum[r] = rs;
}

template <int DT>
__global__ __launch_bounds__(ROW_THREADS) void k_rows(KParams P) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ RowShared sh;
  const int64_t r = blockIdx.x;
  int b, s;
  if (!row_request(P.a, r, b, s)) {
    if (threadIdx.x == 0) P.rowsum[r].mode = M_SKIP;
    return;
  }
  const int mode = row_mode(P.a, b, P.force_greedy);
  switch (mode) {
    case M_GREEDY:
      row_work<DT, M_GREEDY>(P, r, b, s, sh, dyn);
      break;
    case M_LIST:
      row_work<DT, M_LIST>(P, r, b, s, sh, dyn);
      break;
    case M_UNF:
      row_work<DT, M_UNF>(P, r, b, s, sh, dyn);
      break;
    default:
      if constexpr (DT == DSV_BF16)
        row_work<DT, M_HIST>(P, r, b, s, sh, dyn);
      else if (threadIdx.x == 0)
        P.rowsum[r].mode = M_SKIP;  // rejected on the host: float32 nucleus rows
      break;
  }
}

// ---------------------------------------------------------------------------------------
// Rejection walk (shared by k_chunks; sampling/sparse/accept.py:249-283)
// ---------------------------------------------------------------------------------------
__device__ void walk(const KParams& P, int b, int& a_out, int& all_out, int64_t& rstar) {
  const dsv_verify_args& a = P.a;
  const int64_t row0 = request_row0(a, b);
  int cap = req_cap(a, b);
  if (row0 < 0 || row0 >= a.rows) {  // inconsistent row offsets: never read past the rows
    a_out = 0;
    all_out = 1;
    rstar = a.rows > 0 ? a.rows - 1 : 0;
    return;
  }
  if (row0 + cap > a.rows) cap = (int)(a.rows - row0);
  int acc = 0;
  while (acc < cap - 1) {
    const int64_t token = a.candidates[(int64_t)b * a.T + acc + 1];
    const float p = P.rowsum[row0 + acc].p_draft;
    const int64_t qi = ((int64_t)b * (a.T - 1) + acc) * a.K;
    float q = 0.f;
    for (int l = 0; l < a.K; ++l)
      if (load_index(a.q_ids, a.q_ids_i64, qi + l) == token) q += a.q_values[qi + l];
    const float coin = a.uniforms[(int64_t)b * (a.T - 1) + acc];
    if (q > 0.f && q <= 1.f && coin * q < p)
      ++acc;
    else
      break;
  }
  a_out = acc;
  all_out = acc == cap - 1;
  rstar = row0 + acc;
}

// P at one element of a dense-support bonus row (UNF: softmax p; HIST: kept p / S_f).
template <int DT>
__device__ __forceinline__ double dense_P(const RowSum& rs, float T, float x) {
  const float p = prob_of(x, T, rs.m_f, rs.invZ);
  return rs.mode == M_HIST ? (double)(p / rs.S_f) : (double)p;
}

template <int DT>
__global__ __launch_bounds__(CHUNK_THREADS) void k_chunks(KParams P) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[CHUNK_THREADS / WAVE];
  __shared__ int32_t s_a, s_all;
  __shared__ int64_t s_rstar;
  __shared__ int32_t s_qrank[QMAX];
  const dsv_verify_args& a = P.a;
  const int b = blockIdx.y, c = blockIdx.x;
  if (threadIdx.x == 0) {
    int acc, all;
    int64_t rstar;
    walk(P, b, acc, all, rstar);
    s_a = acc;
    s_all = all;
    s_rstar = rstar;
    if (c == 0) P.req[b] = ReqState{acc, all, (int32_t)rstar, P.rowsum[rstar].mode};
  }
  for (int i = threadIdx.x; i < QMAX; i += blockDim.x) s_qrank[i] = 0;
  __syncthreads();
  const int64_t rstar = s_rstar;
  const RowSum rs = P.rowsum[rstar];
  if (rs.mode != M_UNF && rs.mode != M_HIST) return;
  const int64_t V = a.vocab;
  const int64_t lo = (int64_t)c * P.chunk;
  const int64_t hi = lo + P.chunk < V ? lo + P.chunk : V;
  const float T = a.temperatures[b];
  const size_t esize = DT == DSV_BF16 ? 2 : 4;
  const char* rowp = reinterpret_cast<const char*>(a.logits) + (size_t)rstar * (size_t)a.row_stride * esize;
  uint32_t* bm = reinterpret_cast<uint32_t*>(dyn);
  const bool pen = a.hist_ids != nullptr;
  float pres = 0.f, rep = 1.f;
  if (pen) {
    pres = a.presence ? a.presence[b] : 0.f;
    rep = a.repetition ? a.repetition[b] : 1.f;
    build_bitmap(a, b, lo, (int)((P.chunk + 31) / 32), bm);
  }
  // q lanes of the rejected position whose id lies here (for their tie ranks)
  const bool resid = !s_all;
  const int64_t qi = ((int64_t)b * (a.T - 1) + s_a) * a.K;
  double mass = 0.0;
  int32_t ties = 0;
  for (int64_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
    float x = load_elem<DT>(rowp, j);
    if (pen && bitmap_test(bm, j - lo)) x = penalize<DT>(x, pres, rep);
    if (rs.mode == M_UNF) {
      mass += (double)prob_of(x, T, rs.m_f, rs.invZ);
    } else {
      const uint32_t k = key_of<DT>(x);
      if (k > rs.vcut) {
        mass += dense_P<DT>(rs, T, x);
      } else if (k == rs.vcut) {
        ++ties;
        if (resid) {
          for (int l = 0; l < a.K && l < QMAX; ++l) {
            const int64_t id = load_index(a.q_ids, a.q_ids_i64, qi + l);
            if (id > j && id >= lo && id < hi) atomicAdd(&s_qrank[l], 1);
          }
        }
      }
    }
  }
  const double msum = block_sum(mass, red_d);
  const double tsum = block_sum((double)ties, red_d);
  if (threadIdx.x == 0) P.chunks[(int64_t)b * NCH + c] = ChunkSum{msum, (int32_t)tsum, 0};
  if (resid && rs.mode == M_HIST) {
    for (int l = threadIdx.x; l < a.K && l < QMAX; l += blockDim.x) {
      const int64_t id = load_index(a.q_ids, a.q_ids_i64, qi + l);
      if (id >= lo && id < hi) P.qrank[(int64_t)b * QMAX + l] = s_qrank[l];
    }
  }
}

// ---------------------------------------------------------------------------------------
// k_finalize: bonus draw and outputs (sampling/sparse/accept.py:284-307, :179-204, :310-419)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float clamp01(float q) { return (q >= 0.f && q <= 1.f) ? q : 0.f; }

template <int DT>
__global__ __launch_bounds__(CHUNK_THREADS) void k_finalize(KParams P) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[CHUNK_THREADS / WAVE];
  __shared__ double s_prefix, s_thr;
  __shared__ int32_t s_chunk, s_done;
  __shared__ int64_t s_bonus;
  __shared__ int32_t s_tieq;
  const dsv_verify_args& a = P.a;
  const int b = blockIdx.x;
  const ReqState st = P.req[b];
  const int64_t rstar = st.rstar;
  const RowSum rs = P.rowsum[rstar];
  const int64_t V = a.vocab;
  const bool all = st.all != 0;
  const int64_t qi = ((int64_t)b * (a.T - 1) + st.a) * a.K;
  const float uf = a.uniform_final[b];
  const int tid = threadIdx.x;
  if (tid == 0) s_bonus = V - 1;

  if (rs.mode == M_GREEDY || rs.mode == M_LIST) {
    if (tid == 0) {
      const ListEntry* list = P.lists + rstar * DSV_LIST_K;
      double w[DSV_LIST_K];
      double mass = 0.0, pmass = 0.0;
      for (int i = 0; i < rs.nlist; ++i) {
        double Pi = (double)list[i].P;
        double wi = Pi;
        if (!all) {
          float qv = -1.f;  // last lane with this id wins
          for (int l = 0; l < a.K; ++l)
            if (load_index(a.q_ids, a.q_ids_i64, qi + l) == list[i].id) qv = clamp01(a.q_values[qi + l]);
          if (qv >= 0.f) wi = fmax(Pi - (double)qv, 0.0);
        }
        w[i] = wi;
        mass += wi;
        pmass += Pi;
      }
      if (all || mass <= 0.0) {
        for (int i = 0; i < rs.nlist; ++i) w[i] = (double)list[i].P;
        mass = pmass;
      }
      const double thr = (double)uf * mass;
      double cdf = 0.0;
      int64_t bonus = V - 1;
      for (int i = 0; i < rs.nlist; ++i) {
        cdf += w[i];
        if (cdf > thr) {
          bonus = list[i].id;
          break;
        }
      }
      s_bonus = bonus;
    }
    __syncthreads();
  } else {
    // dense support: chunk masses from k_chunks, corrections at the q ids
    const float T = a.temperatures[b];
    const size_t esize = DT == DSV_BF16 ? 2 : 4;
    const char* rowp = reinterpret_cast<const char*>(a.logits) + (size_t)rstar * (size_t)a.row_stride * esize;
    const ChunkSum* cs = P.chunks + (int64_t)b * NCH;
    const bool pen = a.hist_ids != nullptr;
    float pres = 0.f, rep = 1.f;
    uint32_t* bm = reinterpret_cast<uint32_t*>(dyn);
    if (pen) {
      pres = a.presence ? a.presence[b] : 0.f;
      rep = a.repetition ? a.repetition[b] : 1.f;
      build_bitmap(a, b, 0, (int)((V + 31) / 32), bm);
    }
    const int nch = (int)((V + P.chunk - 1) / P.chunk);
    const double P_cut = rs.mode == M_HIST ? dense_P<DT>(rs, T, value_of_key<DT>(rs.vcut)) : 0.0;
    if (tid == 0) {
      // kept mass per chunk (pure), then residual deltas at q ids
      double Mp[NCH], Mr[NCH];
      int32_t tie_prefix[NCH];
      int32_t tp = 0;
      for (int c = 0; c < nch; ++c) {
        tie_prefix[c] = tp;
        int32_t kt = 0;
        if (rs.mode == M_HIST) {
          const int64_t room = (int64_t)rs.ktie - tp;
          kt = room <= 0 ? 0 : (room < cs[c].ties ? (int32_t)room : cs[c].ties);
        }
        tp += cs[c].ties;
        Mp[c] = cs[c].mass + (kt > 0 ? (double)kt * P_cut : 0.0);
        Mr[c] = Mp[c];
      }
      if (!all) {
        for (int l = 0; l < a.K; ++l) {
          const int64_t id = load_index(a.q_ids, a.q_ids_i64, qi + l);
          if (id < 0 || id >= V) continue;
          bool last = true;  // only the last lane with this id counts
          for (int l2 = l + 1; l2 < a.K; ++l2)
            if (load_index(a.q_ids, a.q_ids_i64, qi + l2) == id) last = false;
          if (!last) continue;
          float x = load_elem<DT>(rowp, id);
          if (pen && bitmap_test(bm, id)) x = penalize<DT>(x, pres, rep);
          double Pq = 0.0;
          const int c = (int)(id / P.chunk);
          if (rs.mode == M_UNF) {
            Pq = (double)prob_of(x, T, rs.m_f, rs.invZ);
          } else {
            const uint32_t k = key_of<DT>(x);
            const bool kept = k > rs.vcut ||
                              (k == rs.vcut && (int64_t)tie_prefix[c] + P.qrank[(int64_t)b * QMAX + l] <
                                                   (int64_t)rs.ktie);
            Pq = kept ? dense_P<DT>(rs, T, x) : 0.0;
          }
          const double qv = (double)clamp01(a.q_values[qi + l]);
          const double delta = Pq - fmax(Pq - qv, 0.0);
          Mr[c] -= delta;
        }
      }
      double mp = 0.0, mr = 0.0;
      for (int c = 0; c < nch; ++c) {
        mp += Mp[c];
        mr += Mr[c];
      }
      const bool use_r = !all && mr > 0.0;
      const double mass = use_r ? mr : mp;
      const double thr = (double)uf * mass;
      double pre = 0.0;
      int cstar = -1;
      for (int c = 0; c < nch; ++c) {
        const double mc = use_r ? Mr[c] : Mp[c];
        if (pre + mc > thr) {
          cstar = c;
          break;
        }
        pre += mc;
      }
      s_chunk = cstar;
      s_prefix = pre;
      s_thr = thr;
      s_done = use_r ? 1 : 0;
      s_tieq = cstar >= 0 ? tie_prefix[cstar] : 0;
    }
    __syncthreads();
    // rescan the crossing chunk (and following ones if rounding pushes past its end)
    const bool use_r = s_done != 0;
    for (int c = s_chunk; c >= 0 && c < nch; ++c) {
      const int64_t lo = (int64_t)c * P.chunk;
      const int64_t hi = lo + P.chunk < V ? lo + P.chunk : V;
      const int64_t span = hi - lo;
      const int64_t per = (span + CHUNK_THREADS - 1) / CHUNK_THREADS;
      const int64_t mlo = lo + per * tid;
      const int64_t mhi = mlo + per < hi ? mlo + per : hi;
      // tie prefix inside the chunk (HIST): ties before this thread's sub-range
      int32_t my_ties = 0;
      if (rs.mode == M_HIST) {
        for (int64_t j = mlo; j < mhi; ++j) {
          float x = load_elem<DT>(rowp, j);
          if (pen && bitmap_test(bm, j)) x = penalize<DT>(x, pres, rep);
          my_ties += key_of<DT>(x) == rs.vcut;
        }
      }
      int32_t tie_tot = 0;
      const int32_t tie_before = block_excl_scan(my_ties, reinterpret_cast<int32_t*>(red_d), &tie_tot);
      // per-thread masses
      auto weight = [&](int64_t j, int32_t& tie_seen) -> double {
        float x = load_elem<DT>(rowp, j);
        if (pen && bitmap_test(bm, j)) x = penalize<DT>(x, pres, rep);
        double Pj = 0.0;
        if (rs.mode == M_UNF) {
          Pj = (double)prob_of(x, T, rs.m_f, rs.invZ);
        } else {
          const uint32_t k = key_of<DT>(x);
          bool kept = k > rs.vcut;
          if (k == rs.vcut) {
            kept = (int64_t)s_tieq + tie_before + tie_seen < (int64_t)rs.ktie;
            ++tie_seen;
          }
          Pj = kept ? dense_P<DT>(rs, T, x) : 0.0;
        }
        if (use_r) {
          float qv = -1.f;
          for (int l = 0; l < a.K; ++l)
            if (load_index(a.q_ids, a.q_ids_i64, qi + l) == j) qv = clamp01(a.q_values[qi + l]);
          if (qv >= 0.f) Pj = fmax(Pj - (double)qv, 0.0);
        }
        return Pj;
      };
      double mine = 0.0;
      {
        int32_t seen = 0;
        for (int64_t j = mlo; j < mhi; ++j) mine += weight(j, seen);
      }
      double tot = 0.0;
      const double before = block_excl_scan(mine, red_d, &tot);
      const double thr = s_thr;
      const double pre = s_prefix;
      if (pre + before <= thr && pre + before + mine > thr) {
        double cdf = pre + before;
        int32_t seen = 0;
        for (int64_t j = mlo; j < mhi; ++j) {
          cdf += weight(j, seen);
          if (cdf > thr) {
            s_bonus = j;
            break;
          }
        }
      }
      __syncthreads();
      if (s_bonus != V - 1 || pre + tot > thr) break;
      if (tid == 0) {
        s_prefix = pre + tot;
        s_tieq += tie_tot;
      }
      __syncthreads();
    }
    __syncthreads();
  }

  // ---- outputs ------------------------------------------------------------------------
  const int64_t bonus = s_bonus;
  const int acc = st.a;
  const int T = a.T;
  for (int i = tid; i < T; i += blockDim.x) {
    int64_t v = 0;
    if (i < acc)
      v = a.candidates[(int64_t)b * T + i + 1];
    else if (i == acc)
      v = bonus;
    a.output[(int64_t)b * T + i] = v;
    if (a.kv_slots) {
      int32_t slot = -1;
      if (i <= acc && a.page_table) {
        const int64_t pos = (int64_t)a.prefix_lens[b] + i;
        if (pos >= 0 && pos < a.page_cols) slot = a.page_table[(int64_t)b * a.page_stride + pos];
      }
      a.kv_slots[(int64_t)b * T + i] = slot;
    }
  }
  if (tid == 0) {
    a.accept[b] = acc;
    a.commit[b] = acc + 1;
    a.bonus[b] = bonus;
    a.new_seq[b] = a.prefix_lens[b] + acc + 1;
  }
}

// ---------------------------------------------------------------------------------------
// Greedy verify (verification/caps.py:32-59, verification/ragged.py:51-76)
// ---------------------------------------------------------------------------------------
__global__ void k_greedy_accept(const RowSum* rowsum, const int64_t* cand, const int32_t* lens,
                                int32_t cap_static, const int32_t* prefix, int32_t bs, int32_t T,
                                int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                                int32_t* new_seq, int64_t* top1_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= bs) return;
  int cap = lens ? lens[b] : cap_static;
  cap = cap < 1 ? 1 : (cap > T ? T : cap);
  int acc = cap - 1;
  for (int i = 0; i < cap - 1; ++i) {
    if (cand[(int64_t)b * T + i + 1] != (int64_t)rowsum[(int64_t)b * T + i].argmax) {
      acc = i;
      break;
    }
  }
  const int64_t bon = rowsum[(int64_t)b * T + acc].argmax;
  for (int i = 0; i < T; ++i) {
    const int64_t proposed = i < T - 1 ? cand[(int64_t)b * T + i + 1] : 0;
    output[(int64_t)b * T + i] = i == acc ? bon : proposed;
    if (top1_out) top1_out[(int64_t)b * T + i] = rowsum[(int64_t)b * T + i].argmax;
  }
  accept[b] = acc;
  commit[b] = acc + 1;
  bonus[b] = bon;
  new_seq[b] = prefix[b] + acc + 1;
}

// ---------------------------------------------------------------------------------------
// Top-k rows (kernels/dspine.py:165-207 with the lower-id tie rule)
// ---------------------------------------------------------------------------------------
constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_U = 2;
constexpr int TOPK_BLOCK = TOPK_THREADS * 8 * TOPK_U;

template <int DT>
__global__ __launch_bounds__(TOPK_THREADS) void k_topk(const void* logits, int64_t rows, int64_t V,
                                                       int64_t row_stride, int32_t K, int aligned,
                                                       int cap, float* values_out, int64_t* ids_out,
                                                       int sort_by_id) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t hist256[256];
  __shared__ uint64_t su[16];
  __shared__ int32_t s_cnt, s_cnt2;
  __shared__ uint64_t s_thr;
  uint64_t* cbuf = reinterpret_cast<uint64_t*>(dyn);
  uint64_t* top = cbuf + cap;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
  const size_t esize = DT == DSV_BF16 ? 2 : 4;
  const char* rowp = reinterpret_cast<const char*>(logits) + (size_t)r * (size_t)row_stride * esize;
  if (tid == 0) {
    s_cnt = 0;
    s_thr = 0ull;
  }
  __syncthreads();
  const int64_t NVt = (V + 7) / 8;
  constexpr int U = TOPK_U;
  for (int64_t v0 = 0; v0 < NVt; v0 += (int64_t)TOPK_THREADS * U) {
    Raw<DT> raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + (int64_t)u * TOPK_THREADS + tid;
      if (vi < NVt) load_raw<DT>(raw[u], rowp, vi, V, aligned != 0);
    }
    uint64_t pk[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + (int64_t)u * TOPK_THREADS + tid;
      float x[8];
      if (vi < NVt) decode<DT>(raw[u], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t j = vi * 8 + e;
        pk[u][e] = (vi < NVt && j < V) ? pack(key_of<DT>(x[e]), j) : 0ull;
      }
    }
    if (v0 == 0) {
      uint64_t tm = 0ull;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) tm = pk[u][e] > tm ? pk[u][e] : tm;
      const int J = (K + 15) / 16;
      uint64_t w = 0ull;
      for (int i = 0; i < J; ++i) {
        w = wave_max_u64(tm);
        if (tm == w) tm = 0ull;
      }
      if (lane == 0) su[wid] = w;
      __syncthreads();
      if (tid == 0) {
        uint64_t t0 = ~0ull;
        for (int i = 0; i < TOPK_THREADS / WAVE; ++i) t0 = su[i] < t0 ? su[i] : t0;
        s_thr = t0 ? t0 : 1ull;
      }
      __syncthreads();
    }
    const uint64_t thr = s_thr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool h = pk[u][e] >= thr && pk[u][e] != 0ull;
        const uint64_t bal = __ballot(h);
        if (bal == 0ull) continue;
        const int first = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane == first) base = atomicAdd(&s_cnt, __popcll(bal));
        base = __shfl(base, first, WAVE);
        if (h) {
          const int slot = base + __popcll(bal & ((1ull << lane) - 1ull));
          if (slot < cap) cbuf[slot] = pk[u][e];
        }
      }
    }
    __syncthreads();
    int n = s_cnt < cap ? s_cnt : cap;
    if (v0 == 0 || n > cap - TOPK_BLOCK) {
      const int kk = select_top_fast<DT == DSV_BF16 ? 40 : 56>(cbuf, n, K, top, hist256, su, &s_cnt2);
      if (tid == 0) {
        s_cnt = kk;
        if (kk == K) s_thr = cbuf[K - 1] + 1ull;
      }
      __syncthreads();
    }
  }
  int n = s_cnt < cap ? s_cnt : cap;
  __syncthreads();
  const int kk = select_top_fast<DT == DSV_BF16 ? 40 : 56>(cbuf, n, K, top, hist256, su, &s_cnt2);
  // cbuf[0..kk) sorted (value desc, id asc)
  for (int i = tid; i < K; i += blockDim.x) {
    const bool ok = i < kk;
    const uint64_t v = ok ? cbuf[i] : 0ull;
    const int64_t id = ok ? (int64_t)unpack_id(v) : -1;
    if (values_out) values_out[r * K + i] = ok ? value_of_key<DT>(unpack_key(v)) : -INFINITY;
    if (!sort_by_id) ids_out[r * K + i] = id;
    else top[i] = ok ? (uint64_t)id : ~0ull;
  }
  if (sort_by_id) {
    __syncthreads();
    for (int i = tid; i < K; i += blockDim.x) {
      const uint64_t v = top[i];
      int rank = 0;
      for (int j = 0; j < K; ++j) rank += top[j] < v || (top[j] == v && j < i);
      ids_out[r * K + rank] = v == ~0ull ? -1 : (int64_t)v;
    }
  }
}

}  // namespace dsv

// =========================================================================================
// Host entry points
// =========================================================================================
using namespace dsv;

static int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

struct WsLayout {
  int64_t rowsum, lists, req, chunks, qrank, total;
};
static WsLayout ws_layout(int64_t rows, int32_t bs) {
  WsLayout w;
  int64_t o = 0;
  w.rowsum = o;
  o = align_up(o + rows * (int64_t)sizeof(RowSum), 256);
  w.lists = o;
  o = align_up(o + rows * DSV_LIST_K * (int64_t)sizeof(ListEntry), 256);
  w.req = o;
  o = align_up(o + (int64_t)bs * (int64_t)sizeof(ReqState), 256);
  w.chunks = o;
  o = align_up(o + (int64_t)bs * NCH * (int64_t)sizeof(ChunkSum), 256);
  w.qrank = o;
  o = align_up(o + (int64_t)bs * QMAX * 4, 256);
  w.total = o;
  return w;
}

extern "C" int64_t dsv_verify_workspace_bytes(int64_t rows, int32_t bs, int32_t T, int64_t vocab) {
  (void)T;
  (void)vocab;
  return ws_layout(rows, bs).total;
}

extern "C" int64_t dsv_greedy_workspace_bytes(int64_t rows) { return ws_layout(rows, 1).total; }

static size_t row_lds_bytes(int need_big, int64_t bitmap_words) {
  size_t bytes = need_big ? (size_t)LIST_CAP * 8 : 0;
  if (bitmap_words > 0) bytes = (size_t)LIST_CAP * 8 + (size_t)bitmap_words * 4;
  return bytes;
}

static const size_t LDS_LIMIT = 160 * 1024;

static int launch_rows(const KParams& P, int dtype, int need_big, hipStream_t stream) {
  const dsv_verify_args& a = P.a;
  const size_t lds = row_lds_bytes(need_big, P.bitmap_words);
  if (lds + sizeof(RowShared) > LDS_LIMIT)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "vocab %lld with history penalties needs %zu bytes of LDS (> %zu)",
             (long long)a.vocab, lds + sizeof(RowShared), LDS_LIMIT);
  if (dtype == DSV_BF16) {
    hipFuncSetAttribute((const void*)k_rows<DSV_BF16>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k_rows<DSV_BF16>, dim3((unsigned)a.rows), dim3(ROW_THREADS), lds, stream, P);
  } else {
    hipFuncSetAttribute((const void*)k_rows<DSV_F32>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k_rows<DSV_F32>, dim3((unsigned)a.rows), dim3(ROW_THREADS), lds, stream, P);
  }
  DSV_CHECK_LAUNCH("k_rows");
  return DSV_OK;
}

extern "C" int dsv_verify(const dsv_verify_args* args, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: null arguments");
  const dsv_verify_args& a = *args;
  if (a.logits_dtype != DSV_BF16 && a.logits_dtype != DSV_F32)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: logits must be float32 or bfloat16");
  if (a.bs <= 0 || a.T < 1 || a.vocab < 1 || a.rows < 0 || a.row_stride < a.vocab)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: invalid shape (bs %d, T %d, vocab %lld, rows %lld)", a.bs,
             a.T, (long long)a.vocab, (long long)a.rows);
  if (a.vocab >= (1ll << 31)) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: vocab must be < 2^31");
  if (!a.row_offsets && a.rows != (int64_t)a.bs * a.T)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: dense layout needs rows == bs*T (%lld != %d*%d)",
             (long long)a.rows, a.bs, a.T);
  if (!a.logits || !a.temperatures || !a.top_ks || !a.top_ps || !a.candidates || !a.q_ids ||
      !a.q_values || !a.uniforms || !a.uniform_final || !a.prefix_lens || !a.accept || !a.commit ||
      !a.bonus || !a.output || !a.new_seq || !a.workspace)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: required pointer is null");
  if (a.K < 1 || a.K > QMAX) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: q width K=%d outside [1, %d]", a.K, QMAX);
  if (a.hist_ids && a.hist_len < 0) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: negative hist_len");
  if (a.kv_slots && a.page_table && a.page_cols < 1) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: empty page table");
  if (a.backend != DSV_BACKEND_PYTORCH && a.backend != DSV_BACKEND_FLASHINFER)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: unknown backend %d", a.backend);
  const bool hist_possible = a.filter && a.max_top_k > DSV_LIST_K;
  if (hist_possible && a.logits_dtype != DSV_BF16)
    DSV_FAIL(DSV_ERR_UNSUPPORTED,
             "dsv_verify: float32 logits with top_k > %d (nucleus rows) are not implemented; use bfloat16",
             DSV_LIST_K);
  if (hist_possible && a.backend == DSV_BACKEND_FLASHINFER && a.need_min_p)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_verify: flashinfer min-p branch with top_k > %d is not implemented",
             DSV_LIST_K);
  const WsLayout w = ws_layout(a.rows, a.bs);
  if (a.workspace_bytes < w.total)
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_verify: workspace %lld < %lld bytes", (long long)a.workspace_bytes,
             (long long)w.total);
  const size_t esize = a.logits_dtype == DSV_BF16 ? 2 : 4;
  KParams P;
  P.a = a;
  char* ws = reinterpret_cast<char*>(a.workspace);
  P.rowsum = reinterpret_cast<RowSum*>(ws + w.rowsum);
  P.lists = reinterpret_cast<ListEntry*>(ws + w.lists);
  P.req = reinterpret_cast<ReqState*>(ws + w.req);
  P.chunks = reinterpret_cast<ChunkSum*>(ws + w.chunks);
  P.qrank = reinterpret_cast<int32_t*>(ws + w.qrank);
  P.chunk = align_up((a.vocab + NCH - 1) / NCH, 8);
  P.aligned = ((uintptr_t)a.logits % 16 == 0) && ((a.row_stride * (int64_t)esize) % 16 == 0);
  P.bitmap_words = a.hist_ids && a.hist_len > 0 ? (int32_t)((a.vocab + 31) / 32 + 1) : 0;
  if (!(a.hist_ids && a.hist_len > 0)) P.a.hist_ids = nullptr;
  P.force_greedy = 0;
  P.pad = 0;
  if (a.rows == 0) return DSV_OK;
  const int stages = a.stages ? a.stages : 7;
  const int need_big = a.filter ? 1 : 0;
  if (stages & 1) {
    int rc = launch_rows(P, a.logits_dtype, need_big, stream);
    if (rc) return rc;
  }
  if (!(stages & 6)) return DSV_OK;
  const size_t chunk_lds = P.a.hist_ids ? (size_t)((P.chunk + 31) / 32) * 4 : 0;
  if (a.logits_dtype == DSV_BF16)
    hipLaunchKernelGGL(k_chunks<DSV_BF16>, dim3(NCH, a.bs), dim3(CHUNK_THREADS), chunk_lds, stream, P);
  else
    hipLaunchKernelGGL(k_chunks<DSV_F32>, dim3(NCH, a.bs), dim3(CHUNK_THREADS), chunk_lds, stream, P);
  DSV_CHECK_LAUNCH("k_chunks");
  if (!(stages & 4)) return DSV_OK;
  const size_t fin_lds = P.a.hist_ids ? (size_t)((a.vocab + 31) / 32) * 4 : 0;
  if (fin_lds > 64 * 1024) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_verify: vocab too large for the penalty bitmap");
  if (a.logits_dtype == DSV_BF16)
    hipLaunchKernelGGL(k_finalize<DSV_BF16>, dim3(a.bs), dim3(CHUNK_THREADS), fin_lds, stream, P);
  else
    hipLaunchKernelGGL(k_finalize<DSV_F32>, dim3(a.bs), dim3(CHUNK_THREADS), fin_lds, stream, P);
  DSV_CHECK_LAUNCH("k_finalize");
  return DSV_OK;
}

extern "C" int dsv_greedy_verify(const void* logits, int32_t dtype, int64_t rows, int64_t vocab,
                                 int64_t row_stride, int32_t bs, int32_t T, const int64_t* candidates,
                                 const int32_t* verify_lens, int32_t cap, const int32_t* prefix_lens,
                                 int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                                 int32_t* new_seq, int64_t* top1_out, void* workspace,
                                 int64_t workspace_bytes, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (dtype != DSV_BF16 && dtype != DSV_F32)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify: logits must be float32 or bfloat16");
  if (bs <= 0 || T < 1 || vocab < 1 || row_stride < vocab || rows != (int64_t)bs * T)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify: logits must be [bs*T, V] (rows %lld, bs %d, T %d)",
             (long long)rows, bs, T);
  if (!verify_lens && (cap < 1 || cap > T))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify: cap %d outside [1, %d]", cap, T);
  if (!logits || !candidates || !prefix_lens || !accept || !commit || !bonus || !output || !new_seq ||
      !workspace)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify: required pointer is null");
  const WsLayout w = ws_layout(rows, 1);
  if (workspace_bytes < w.total)
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_greedy_verify: workspace %lld < %lld", (long long)workspace_bytes,
             (long long)w.total);
  const size_t esize = dtype == DSV_BF16 ? 2 : 4;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.a.logits = logits;
  P.a.logits_dtype = dtype;
  P.a.rows = rows;
  P.a.vocab = vocab;
  P.a.row_stride = row_stride;
  P.a.bs = bs;
  P.a.T = T;
  P.a.verify_lens = nullptr;  // every row's argmax is reported
  P.a.candidates = candidates;
  char* ws = reinterpret_cast<char*>(workspace);
  P.rowsum = reinterpret_cast<RowSum*>(ws + w.rowsum);
  P.lists = reinterpret_cast<ListEntry*>(ws + w.lists);
  P.aligned = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esize) % 16 == 0);
  P.force_greedy = 1;
  int rc = launch_rows(P, dtype, 0, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(k_greedy_accept, dim3((bs + 63) / 64), dim3(64), 0, stream, P.rowsum, candidates,
                     verify_lens, cap, prefix_lens, bs, T, accept, commit, bonus, output, new_seq, top1_out);
  DSV_CHECK_LAUNCH("k_greedy_accept");
  return DSV_OK;
}

extern "C" int dsv_topk(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                        int32_t k, float* values_out, int64_t* ids_out, int32_t sort_by_id,
                        dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (dtype != DSV_BF16 && dtype != DSV_F32)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: logits must be float32 or bfloat16");
  if (rows < 0 || vocab < 1 || row_stride < vocab)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: invalid shape");
  if (k < 1 || k > 1024 || k > vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: k=%d outside [1, min(1024, V)]", k);
  if (!logits || !ids_out) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: null pointer");
  if (rows == 0) return DSV_OK;
  const size_t esize = dtype == DSV_BF16 ? 2 : 4;
  const int aligned = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esize) % 16 == 0);
  const int cap = TOPK_BLOCK + (k > 256 ? k : 256);
  const size_t lds = (size_t)(cap + k) * 8;
  if (lds > 150 * 1024) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_topk: k=%d needs too much LDS", k);
  if (dtype == DSV_BF16) {
    hipFuncSetAttribute((const void*)k_topk<DSV_BF16>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k_topk<DSV_BF16>, dim3((unsigned)rows), dim3(TOPK_THREADS), lds, stream, logits, rows,
                       vocab, row_stride, k, aligned, cap, values_out, ids_out, sort_by_id);
  } else {
    hipFuncSetAttribute((const void*)k_topk<DSV_F32>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(k_topk<DSV_F32>, dim3((unsigned)rows), dim3(TOPK_THREADS), lds, stream, logits, rows,
                       vocab, row_stride, k, aligned, cap, values_out, ids_out, sort_by_id);
  }
  DSV_CHECK_LAUNCH("k_topk");
  return DSV_OK;
}
