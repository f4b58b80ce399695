// Sampled draft verification for gfx950: target distribution, chain rejection with sparse q,
// residual resample, accepted-prefix compaction and KV-slot gather.
//
// Launches of one verify step (no host synchronisation):
//   k_chunk  (rows x C)         every row, in chunks of 20480 bf16 / 12288 fp32 values held in
//                               registers: penalties (the chunk's slice of the request's history
//                               bitmap built in LDS), max/argmax, softmax partial sums, exact
//                               top-k candidates, nucleus value counts -- one read of the logits
//   k_merge  (rows)             per row: Z, the filtered top-k support (id, P), P at the draft
//                               token and the step's accept/reject decision; nucleus rows (a
//                               top-p / min-p cut with top-k > 64) find their cut from the chunk
//                               pass's value counts.  Then the bonus draw the row would give as
//                               the accepted length: drawn for support-list rows, planned (the
//                               chunk and threshold) for dense rows.  The workgroup that merges a
//                               request's last row writes the request's outputs when its accepted
//                               row drew the token.
//   k_final  (requests)         the requests left (launched when a dense row can occur): rows
//                               the counts did not settle first (the full 65536-key histogram, or
//                               the float32 radix descent, in the workgroup's LDS), then the
//                               accepted length, the bonus token of that row (a dense row's
//                               planned chunk scanned here), outputs and KV slots
// The target-distribution entry runs k_chunk, k_merge, then k_nuc over the rows the merge
// listed and k_dense_p.
// Hand-offs between workgroups: kernel boundaries, except the per-request count in k_merge,
// which uses device-coherent stores and loads (no device-scope fence: on this multi-XCD part
// that writes back and invalidates the whole L2).
//
// Semantics follow runtime/worker.py:440-508 (target P, pytorch backend), sampling/rejection.py
// :36-98 and sampling/sparse/accept.py:239-307 (chain rejection and residual resample).
#include <float.h>
#include <string.h>

#include <mutex>

#include <type_traits>

#include "dsv_device.h"

namespace dsv {


struct KParams {
  dsv_verify_args a;
  RowSum* rowsum;         // [rows]
  ListEntry* lists;       // [rows, DSV_LIST_K]
  ChunkStat* cstat;       // [rows, C]
  uint64_t* cand;         // [rows, C, kcand]
  int64_t* rbonus;        // [rows]: the bonus token each row gives as the accepted length
  int32_t* rties;         // [rows, NCHK]: nucleus rows' chunk counts of values at the cut key
  struct DrawPlan* plans; // [rows]: dense rows' planned bonus draw
  int32_t* step_ok;       // [rows]: 1 when the draft token verified by the row is accepted
  uint32_t* pbits;        // [bs, pwords]: history bitmap of each request, NULL without history
  uint32_t* hpart;        // [rows, C, HWIN / 2]: nucleus rows' per-chunk window counts (16-bit pairs)
  uint32_t* nhist;        // [max(NUC_GRID, bs), 65536]: full-histogram counts, one area per workgroup
  int32_t* nuc_rows;      // [rows + 1]: the number of full-histogram rows, then their ids
  int64_t pwords;
  int32_t C;              // chunks per row
  int32_t kcand;          // candidate slots per chunk
  int32_t aligned;        // logits rows are 16-byte aligned
  int32_t force_greedy;   // greedy-verify entry: every row is GREEDY
  int32_t softmax;        // chunk pass computes softmax partial sums (the verify entry)
  int32_t raw_p;          // dense target writer: the filtered p, not renormalised
  int32_t final_nuc;      // k_final resolves the full-histogram rows (no k_nuc launch)
  uint32_t* req_cnt;      // [bs]: rows merged per request (zeroed by the chunk pass)
  uint32_t* deferred;     // [bs]: 1 until the row merge wrote the request's outputs (set by the chunk pass)
  int32_t only_deferred;  // k_final skips the requests the row merge finished
  const float* src_p;     // dense target writer with raw_p: kept entries are src_p's values (the
  int64_t src_stride;     //   probabilities whose logs are the rows: dsv_filter_probs), else NULL
};

__device__ __forceinline__ const char* row_ptr(const dsv_verify_args& a, int64_t r) {
  const size_t esize = a.logits_dtype == DSV_BF16 ? 2 : 4;
  return reinterpret_cast<const char*>(a.logits) + (size_t)r * (size_t)a.row_stride * esize;
}

// The draft token verified by row (b, s), or -1 when the row verifies no step.
__device__ __forceinline__ int64_t step_token(const dsv_verify_args& a, int b, int s) {
  if (!a.candidates) return -1;  // target-distribution entry: no drafts
  const int cap = req_cap(a, b);
  return (s < cap - 1 && s + 1 < a.T) ? a.candidates[(int64_t)b * a.T + s + 1] : -1;
}

// History bits of request b: bit j is set when token j is in the history.
__device__ __forceinline__ uint32_t pen_word(const KParams& P, int b, int64_t w) {
  return P.pbits[(int64_t)b * P.pwords + w];
}
// Bits of tokens [j, j + n) for j a multiple of n and n in {4, 8}.
__device__ __forceinline__ uint32_t pen_bits(const KParams& P, int b, int64_t j, int n) {
  return (pen_word(P, b, j >> 5) >> (j & 31)) & ((1u << n) - 1u);
}
__device__ __forceinline__ bool pen_test(const KParams& P, int b, int64_t j) {
  return (pen_word(P, b, j >> 5) >> (j & 31)) & 1u;
}

// ---------------------------------------------------------------------------------------
// Candidate refill: the chunk holds more values at or above the admission bound than the
// LDS buffer (cbits: the chunk's history bits, lo a multiple of 32).  The K-th largest buffered
// value is a higher bound; re-read the chunk from
// memory until the admitted values fit.  Each raise drops at least CAND_CAP - K >= 256 of the
// buffered values, so a chunk of at most 20480 values needs at most 80 rounds.  With thr0
// nonzero the buffer holds nothing yet and the first read admits the values >= thr0.
// ---------------------------------------------------------------------------------------
template <int DT>
__device__ __noinline__ int refill_candidates(const uint32_t* cbits, const char* rowp, int64_t lo, int64_t hi,
                                              int K, float pres, float rep, uint64_t* cbuf, uint32_t* hist256,
                                              uint64_t* su, int32_t* cnt, uint64_t thr0) {
  constexpr int TOP_SHIFT = DT == DSV_BF16 ? 40 : 56;
  int nb = CAND_CAP + 1;
  for (int iter = 0; iter < 128 && nb > CAND_CAP; ++iter) {
    if (threadIdx.x < WAVE) {
      const uint64_t t = (iter == 0 && thr0) ? thr0 : wave_kth_largest(cbuf, CAND_CAP, K, hist256, TOP_SHIFT);
      if (threadIdx.x == 0) {
        su[0] = t;
        *cnt = 0;
      }
    }
    __syncthreads();
    const uint64_t thr = su[0];
    for (int64_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
      float x = load_elem<DT>(rowp, j);
      if (cbits && ((cbits[(j - lo) >> 5] >> (j & 31)) & 1u)) x = penalize<DT>(x, pres, rep);
      const uint64_t pk = pack(key_of<DT>(x), j);
      if (pk >= thr) {
        const int slot = atomicAdd(cnt, 1);
        if (slot < CAND_CAP) cbuf[slot] = pk;
      }
    }
    __syncthreads();
    nb = *cnt;
    __syncthreads();
  }
  return nb < CAND_CAP ? nb : CAND_CAP;
}

// The thread's share of the chunk's values whose key is `key` (cbits: the chunk's history bits),
// re-read from memory: the tie count of a sparse joint row's chunk whose candidate buffer was
// refilled.
template <int DT>
__device__ __noinline__ int count_key_chunk(const uint32_t* cbits, const char* rowp, int64_t lo, int64_t hi,
                                            uint32_t key, float pres, float rep) {
  int cnt = 0;
  for (int64_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
    float x = load_elem<DT>(rowp, j);
    if (cbits && ((cbits[(j - lo) >> 5] >> (j & 31)) & 1u)) x = penalize<DT>(x, pres, rep);
    cnt += key_of<DT>(x) == key;
  }
  return cnt;
}

// ---------------------------------------------------------------------------------------
// Bonus draw machinery (used by the row merge and k_final; see the bonus section below)
// ---------------------------------------------------------------------------------------
constexpr int FCT = 512;      // threads of k_final
constexpr int KF_ROLES = 4;   // k_final workgroups a request: the request's own and three helpers
constexpr int DNW_MAX = FCT / WAVE;
constexpr int64_t BONUS_LATER = -2;  // rbonus: the row is drawn in k_final
// rbonus <= BONUS_PLAN: the row's draw is planned; the request's final scans chunk
// BONUS_PLAN - 1 - rbonus (-1: no mass anywhere, no scan)
constexpr int64_t BONUS_PLAN = -3;
// deferred[b]: 0 done, 1 k_final decides the request, else a planned draw at accepted length
// (deferred & (DEFER_ACC - 1)) - 2 in chunk (deferred >> 24) - 1
constexpr int DEFER_ACC = 1 << 24;

struct DrawShared {
  double red_d[DNW_MAX];
  int32_t red_i[DNW_MAX];
  uint64_t red_u[DNW_MAX];
  int64_t qid[QMAX];
  float qv[QMAX];       // clamped q of the lane
  float qraw[QMAX];     // q of the lane as given (the draft test sums these)
  int32_t qlast[QMAX];  // lane is the last one with its id (its q is the residual's)
  int32_t qrank[QMAX];  // q id at a split cut key: values at the cut key before it (id order), else -1
  float qx[QMAX];       // adjusted value at the q id
  double qd[QMAX];      // P - max(P - q, 0) at a q id (the residual's reduction), else 0
  double cm[NCHK];      // chunk masses of P above the cut (every id of an unfiltered row)
  int32_t ct[NCHK];     // chunk counts of values at the cut key
  ListEntry lst[DSV_LIST_K];  // a support-list row's entries, sorted by id
  int32_t nlist;
  int64_t bonus;
  double chunk_lo, thr, pick_lo;
  int32_t acc, chunk, tieq, use_r, pick_thread, ptb;
  uint64_t rmask;    // q lanes that need their rank at a split cut key
  uint64_t qmask;    // residual q lanes whose id lies in the planned chunk
  uint4 pv[CV_MAX];   // the picked thread's span (penalised)
};

// The draw's P at value x: exp2(x c2 - M c2) * scale, scale = 1/Z (over the kept mass S for a
// filtered row).
struct BonusP {
  float c2, mc2, scale;
  __device__ __forceinline__ float operator()(float x) const {
    return __builtin_amdgcn_exp2f(fmaf(x, c2, -mc2)) * scale;
  }
};
template <int DT>
__device__ __forceinline__ BonusP bonus_p(const RowSum& rs, float T) {
  BonusP q;
  q.c2 = log2e_over(T);
  q.mc2 = value_of_key<DT>(rs.kmax) * q.c2;
  q.scale = rs.invZ * ((rs.mode == M_HIST || rs.norm) ? 1.f / rs.S_f : 1.f);
  return q;
}

// Stage the sparse q of draft step `step` of request b (live = false: no q): ids, clamped
// values, and which lane of a repeated id carries the residual's q (the last one).
__device__ __forceinline__ void stage_q(const dsv_verify_args& a, int b, int step, bool live, DrawShared& sh) {
  const int tid = threadIdx.x;
  const int64_t qi = ((int64_t)b * (a.T - 1) + step) * a.K;
  for (int l = tid; l < QMAX; l += blockDim.x) {
    const bool on = live && l < a.K;
    sh.qid[l] = on ? load_index(a.q_ids, a.q_ids_i64, qi + l) : -1;
    sh.qv[l] = on ? clamp01(a.q_values[qi + l]) : 0.f;
    sh.qd[l] = 0.0;
    sh.qrank[l] = -1;
  }
  __syncthreads();
  for (int l = tid; l < QMAX; l += blockDim.x) {
    bool last = sh.qid[l] >= 0 && sh.qid[l] < a.vocab;
    for (int l2 = l + 1; l2 < a.K && last; ++l2) last = sh.qid[l2] != sh.qid[l];
    sh.qlast[l] = last;
  }
  __syncthreads();
}

// (one wave, lanes holding q lanes) whether the lane's id is a valid token that no later lane of
// the first K repeats: its q is the one the residual uses
__device__ __forceinline__ bool q_last_lane(int64_t qid, int K, int64_t V) {
  const int lane = threadIdx.x & (WAVE - 1);
  bool last = qid >= 0 && qid < V;
  for (int l2 = 1; l2 < K; ++l2) last = last && !(l2 > lane && readlane_at(qid, l2) == qid);
  return last;
}

// The logit and history word at a q lane's id, loaded by fetch_q_wave and left in flight until
// qx_finish penalises them into sh.qx (the row merge runs in between).
struct QxLoad {
  uint32_t xb;  // the logit's bits at the id (bf16: the 16 bits; -inf without an id)
  uint32_t hw;  // the history word holding the id's bit (0 without a history)
};

// The q lanes of draft step+1 for one wave (lanes are the q lanes): ids, given and clamped
// values, whether the lane is the last with its id -- left in sh, which the workgroup sees after
// a barrier -- and, want_x, the loads of the logit at each such id (ql, for qx_finish).
template <int DT>
__device__ __forceinline__ void fetch_q_wave(const KParams& P, int b, int step, bool live, const char* rowp,
                                             bool want_x, DrawShared& sh, QxLoad& ql) {
  const dsv_verify_args& a = P.a;
  const int lane = threadIdx.x & (WAVE - 1);
  const bool on = live && lane < a.K;
  // loaded whether or not the row tests a draft (its step and lane clamped into the request's
  // q rows), so that the loads do not wait for the request's verify length
  int64_t qid_l = -1;
  float qr_l = 0.f;
  if (a.candidates && a.q_ids && a.q_values && a.T >= 2 && a.K >= 1) {
    const int st = step < a.T - 1 ? step : a.T - 2;
    const int64_t qs = ((int64_t)b * (a.T - 1) + st) * a.K + (lane < a.K ? lane : 0);
    qid_l = load_index(a.q_ids, a.q_ids_i64, qs);
    qr_l = a.q_values[qs];
  }
  const int64_t qid = on ? qid_l : -1;
  const float qr = on ? qr_l : 0.f;
  sh.qid[lane] = qid;
  sh.qraw[lane] = qr;
  sh.qv[lane] = clamp01(qr);
  sh.qd[lane] = 0.0;
  sh.qrank[lane] = -1;
  const bool last = q_last_lane(qid, a.K, a.vocab);
  sh.qlast[lane] = last;
  // raw bits: a conversion here would wait for the load
  ql.xb = DT == DSV_BF16 ? 0xff80u : 0xff800000u;
  ql.hw = 0u;
  if (want_x && last) {
    if constexpr (DT == DSV_BF16)
      ql.xb = reinterpret_cast<const uint16_t*>(rowp)[qid];
    else
      ql.xb = reinterpret_cast<const uint32_t*>(rowp)[qid];
    if (P.pbits) ql.hw = pen_word(P, b, qid >> 5);
  }
}

// The adjusted logit at each q lane's id into sh.qx (the wave that called fetch_q_wave; pres /
// rep: the request's penalties).
template <int DT>
__device__ __forceinline__ void qx_finish(const QxLoad& ql, float pres, float rep, DrawShared& sh) {
  const int lane = threadIdx.x & (WAVE - 1);
  float xq = DT == DSV_BF16 ? bf16_bits_to_f32((uint16_t)ql.xb) : __uint_as_float(ql.xb);
  if ((ql.hw >> (sh.qid[lane] & 31)) & 1u) xq = penalize<DT>(xq, pres, rep);
  sh.qx[lane] = xq;
}

// The draft test from the fetched q lanes (wave-level): q = the sum of the lanes holding tok.
__device__ __forceinline__ int32_t step_accept_lds(const DrawShared& sh, int K, int64_t tok, float p, float coin) {
  const int lane = threadIdx.x & (WAVE - 1);
  uint64_t bal = __ballot(lane < K && sh.qid[lane] == tok);
  float q = 0.f;
  while (bal) {
    const int l = __ffsll((long long)bal) - 1;
    bal &= bal - 1ull;
    q += sh.qraw[l];
  }
  return (q > 0.f && q <= 1.f && coin * q < p) ? 1 : 0;
}

// The row's chunk statistics, draft token and coin, read at the start of the row merge.
struct RowPre {
  ChunkStat cs[NCHK];
  int64_t tok;  // draft token the row tests, -1 for none
  float u;      // its coin
  float uf;     // the request's bonus coin
  float top_p, min_p;
  float pres, rep;  // the request's penalties (0 and 1 without a history)
  int32_t top_k;
};

// History hits of a thread's vectors, penalised in place (about 0.3% of the values): each lane
// copies its vectors holding hits to the wave's LDS slots wv / wm (WHITV of them), one lane per
// copied vector penalises the hit elements there, and the owners read the vectors back -- the
// registers end up penalised without a run-time register index.  bits[u]: the hit elements of
// v[u].  Called by every lane of the wave.
template <int DT, int NV>
__device__ __forceinline__ void penalize_hits(uint4 (&v)[NV], const uint32_t (&bits)[NV], float pres, float rep,
                                              uint4* wv, uint32_t* wm) {
  const int lane = threadIdx.x & (WAVE - 1);
  int hv = 0;
#pragma unroll
  for (int u = 0; u < NV; ++u) hv += bits[u] != 0u;
  // exclusive prefix and total of the hit vectors over the wave (a DPP scan)
  const int incl = wave_incl_scan(hv);
  const int tot = readlane<WAVE - 1>(incl);
  // rounds of the wave's LDS slots (one unless the history is long): the round's hit vectors
  // are copied out, one lane per vector penalises their elements, the owners read them back
  for (int r0 = 0; r0 < tot; r0 += WHITV) {
    int slot = incl - hv - r0;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      if (bits[u]) {
        if ((unsigned)slot < (unsigned)WHITV) {
          wv[slot] = v[u];
          wm[slot] = bits[u];
        }
        ++slot;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nv = tot - r0 < WHITV ? tot - r0 : WHITV;
    for (int i = lane; i < nv; i += WAVE) {
      uint32_t m = wm[i];
      while (m) {
        const int e = __ffs(m) - 1;
        m &= m - 1u;
        if constexpr (DT == DSV_BF16) {
          uint16_t* el = reinterpret_cast<uint16_t*>(&wv[i]) + e;
          *el = (uint16_t)(__float_as_uint(penalize<DT>(bf16_bits_to_f32(*el), pres, rep)) >> 16);
        } else {
          float* el = reinterpret_cast<float*>(&wv[i]) + e;
          *el = penalize<DT>(*el, pres, rep);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    slot = incl - hv - r0;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      if (bits[u]) {
        if ((unsigned)slot < (unsigned)WHITV) v[u] = wv[slot];
        ++slot;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Thread t's span of chunk c in id order (NT threads tile the chunk: ids c*chunk + t*FE + [0,
// FE)): its vectors and history bits, loaded by span_load and handed out penalised, in id
// order, by span_each as f(i, x); -inf past the row.
template <int DT, int NT>
struct Span {
  static constexpr int SV = CT * Elems<DT>::cv / NT, FE = SV * Elems<DT>::n;  // vectors and ids a thread
  uint4 v[SV];
  uint64_t blo, bhi;  // the span's history bits (tokens >= vocab have none)
};
template <int DT, bool ALIGNED, int NT>
__device__ __forceinline__ void span_load(const KParams& P, int b, const char* rowp, int c, Span<DT, NT>& sp) {
  constexpr int n = Elems<DT>::n, CHE = Elems<DT>::chunk;
  constexpr int SV = Span<DT, NT>::SV;
  static_assert(SV * NT == CT * Elems<DT>::cv && Span<DT, NT>::FE <= 96, "spans tile a chunk");
  const int64_t V = P.a.vocab;
  const int64_t clo = (int64_t)c * CHE, chi = clo + CHE < V ? clo + CHE : V;
  const int64_t jlo = clo + (int64_t)threadIdx.x * Span<DT, NT>::FE;
  if constexpr (ALIGNED) {
    const auto rsr = buf_rsrc(rowp + clo * (16 / n), (uint32_t)((chi - clo) * (16 / n)));
#pragma unroll
    for (int u = 0; u < SV; ++u) sp.v[u] = buf_load16(rsr, (uint32_t)threadIdx.x * (SV * 16u), (uint32_t)(u * 16));
#pragma unroll
    for (int u = 0; u < SV; ++u)  // past the row: the buffer reads zeros; -inf and the partial last vector
      if (jlo + u * n + n > chi) sp.v[u] = load_vec<DT>(rowp, jlo / n + u, chi, false);
  } else {
#pragma unroll
    for (int u = 0; u < SV; ++u) sp.v[u] = load_vec<DT>(rowp, jlo / n + u, chi, false);
  }
  sp.blo = 0;
  sp.bhi = 0;
  if (P.pbits) {
    const auto rb = buf_rsrc(P.pbits + (int64_t)b * P.pwords, (uint32_t)(P.pwords * 4));
    const uint32_t w0 = (uint32_t)(jlo >> 5) * 4u, sh = (uint32_t)(jlo & 31);
    const uint64_t A = (uint64_t)buf_load4(rb, w0, 0) | ((uint64_t)buf_load4(rb, w0, 4) << 32);
    const uint64_t B = (uint64_t)buf_load4(rb, w0, 8) | ((uint64_t)buf_load4(rb, w0, 12) << 32);
    sp.blo = (A >> sh) | (sh ? B << (64 - sh) : 0ull);
    sp.bhi = B >> sh;
  }
}
template <int DT, int NT, class F>
__device__ __forceinline__ void span_each(const Span<DT, NT>& sp, float pres, float rep, F&& f) {
  constexpr int n = Elems<DT>::n;
#pragma unroll
  for (int u = 0; u < Span<DT, NT>::SV; ++u)
#pragma unroll
    for (int e = 0; e < n; ++e) {
      const int i = u * n + e;
      float x = vec_elem<DT>(sp.v[u], e);
      if (((i < 64 ? sp.blo >> i : sp.bhi >> (i - 64)) & 1ull)) x = penalize<DT>(x, pres, rep);
      f(i, x);
    }
}
template <int DT, bool ALIGNED, int NT, class F>
__device__ __forceinline__ void for_span(const KParams& P, int b, const char* rowp, int c, float pres, float rep,
                                         F&& f) {
  Span<DT, NT> sp;
  span_load<DT, ALIGNED, NT>(P, b, rowp, c, sp);
  span_each<DT, NT>(sp, pres, rep, f);
}

// Support-list draw (wave 0): entries sh.lst[0, sh.nlist) sorted by id; q staged when resid.
// Sparse joint rows are packed P in the reference: the residual at an id subtracts the clamped q
// of every lane holding it (sampling/sparse/accept.py:186-193); other rows the last lane's.
__device__ __forceinline__ int64_t list_draw(const dsv_verify_args& a, bool resid, float uf, const DrawShared& sh) {
  const int lane = threadIdx.x & (WAVE - 1);
  const bool live = lane < sh.nlist;
  const ListEntry e = live ? sh.lst[lane] : ListEntry{INT_MAX, 0.f};
  const double Pi = (double)e.P;
  double w = Pi;
  if (resid && live) {
    double qs = 0.0;
    for (int l = 0; l < a.K; ++l)
      if (sh.qid[l] == (int64_t)e.id && (a.sparse_joint || sh.qlast[l])) qs += (double)sh.qv[l];
    w = fmax(Pi - qs, 0.0);
  }
  double lo, hi;
  double mass = wave_tiles(w, lo, hi);
  if (!resid || !(mass > 0.0)) mass = wave_tiles(Pi, lo, hi);
  const double thr = (double)uf * mass;
  const uint64_t hit = __ballot(live && lo <= thr && thr < hi);
  return hit ? readlane_at((int64_t)e.id, __ffsll((long long)hit) - 1) : a.vocab - 1;
}

// What a dense row's draw needs after the chunk is known (the row merge writes it; the request's
// final reads it for the accepted row).
struct DrawPlan {
  double thr, chunk_lo;  // the threshold u * mass and the mass before the chunk
  int32_t chunk, tieq;   // the chunk (-1: no mass anywhere) and the cut-key values before it
  int32_t use_r, pad;    // residual (1) or P (0)
  double qd[QMAX];       // the residual's reduction at each q lane
};

// (rare) the rank of q id l among the values of the cut key: the values of that key ahead of it
// in its chunk, over the workgroup, plus the cut-key counts of the chunks before (thread 0 writes
// sh.qrank[l]).
template <int DT, bool ALIGNED, int NT>
__device__ __forceinline__ void q_cut_rank(const KParams& P, int b, const char* rowp, uint32_t vcut, float pres,
                                           float rep, int l, DrawShared& sh) {
  constexpr int NW = NT / WAVE;
  constexpr int n = Elems<DT>::n, CHE = Elems<DT>::chunk;
  const int64_t qid = sh.qid[l];
  const int cq = (int)(qid / CHE);
  const int64_t clo = (int64_t)cq * CHE;
  const int64_t chi = clo + CHE < P.a.vocab ? clo + CHE : P.a.vocab;
  int32_t before = 0;
  // one vector at a time (a rare path: few registers), the values at the cut key before qid
#pragma unroll 1
  for (int64_t vi = clo / n + threadIdx.x; vi * n < qid; vi += NT) {
    const uint4 w = load_vec<DT>(rowp, vi, chi, ALIGNED);
    const uint32_t bits = P.pbits ? pen_bits(P, b, vi * n, n) : 0u;
#pragma unroll
    for (int e = 0; e < n; ++e) {
      float x = vec_elem<DT>(w, e);
      if ((bits >> e) & 1u) x = penalize<DT>(x, pres, rep);
      before += (key_of<DT>(x) == vcut) & (vi * n + e < qid);
    }
  }
  before = block_sum<NW>(before, sh.red_i);
  if (threadIdx.x == 0) {
    for (int c = 0; c < cq; ++c) before += sh.ct[c];
    sh.qrank[l] = before;
  }
  __syncthreads();
}

// Dense draw, first part, over the NT threads of the workgroup: sh.cm / sh.ct hold the chunk
// masses and cut counts, q is staged when resid.  Leaves the plan in sh (chunk, thr, chunk_lo,
// tieq, use_r, qd).
template <int DT, bool ALIGNED, int NT>
__device__ __forceinline__ void dense_plan(const KParams& P, int b, const char* rowp, const RowSum& rs, float T,
                                           float pres, float rep, bool resid, float uf, DrawShared& sh,
                                           bool have_qx = false) {
  constexpr int CHE = Elems<DT>::chunk;
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int C = P.C;
  const bool pen = P.pbits != nullptr;
  const bool hist = rs.mode == M_HIST;
  const bool tie_cut = hist && rs.ktie > 0 && rs.ktie != INT_MAX;  // the cut splits a key's values
  // the q ids' adjusted values; ids at a split cut key need their rank among its values
  int32_t qc = -1;  // (wave 0) the chunk of the lane's residual q id
  if (tid < WAVE) {
    const bool qlive = resid && lane < a.K && sh.qlast[lane];
    float xq = -INFINITY;
    if (have_qx) {  // fetched with the q lanes
      xq = qlive ? sh.qx[lane] : -INFINITY;
    } else if (qlive) {
      const int64_t qid = sh.qid[lane];
      xq = load_elem<DT>(rowp, qid);
      if (pen && pen_test(P, b, qid)) xq = penalize<DT>(xq, pres, rep);
    }
    const bool need = qlive && tie_cut && key_of<DT>(xq) == rs.vcut;
    if (qlive) qc = (int32_t)(sh.qid[lane] / CHE);
    if (lane < QMAX) {
      sh.qx[lane] = xq;
      sh.qrank[lane] = need ? 0 : -1;
    }
    const uint64_t rk = __ballot(need);
    if (lane == 0) sh.rmask = rk;
  }
  __syncthreads();
  for (uint64_t m = sh.rmask; m; m &= m - 1ull)  // (rare) rank of a q id among the cut key's values
    q_cut_rank<DT, ALIGNED, NT>(P, b, rowp, rs.vcut, pres, rep, __ffsll((long long)m) - 1, sh);
  const BonusP bp = bonus_p<DT>(rs, T);
  const double P_cut = hist ? (double)bp(value_of_key<DT>(rs.vcut)) : 0.0;
  if (tid < WAVE) {
    // the residual's reduction at each q id (lanes hold the q lanes)
    double qd = 0.0;
    if (qc >= 0) {
      const float xq = sh.qx[lane];
      const uint32_t k = key_of<DT>(xq);
      const bool kept = !hist || k > rs.vcut ||
                        (k == rs.vcut && (rs.ktie == INT_MAX || (sh.qrank[lane] >= 0 && sh.qrank[lane] < rs.ktie)));
      const double Pq = kept ? (double)bp(xq) : 0.0;
      qd = Pq - fmax(Pq - (double)sh.qv[lane], 0.0);
    }
    if (lane < QMAX) sh.qd[lane] = qd;
    // lanes hold the chunks: masses with the kept values at the cut key, then the residual's
    const int32_t ctl = lane < C ? sh.ct[lane] : 0;
    const int32_t tie_prefix = wave_incl_scan(ctl) - ctl;
    int32_t kt = 0;
    if (hist) {
      const int64_t room = (int64_t)rs.ktie - tie_prefix;
      kt = room <= 0 ? 0 : (room < ctl ? (int32_t)room : ctl);
    }
    const double Mp = lane < C ? sh.cm[lane] + (kt > 0 ? (double)kt * P_cut : 0.0) : 0.0;
    double Mr = Mp;
    for (uint64_t m = __ballot(qc >= 0); m; m &= m - 1ull) {  // (q lanes in id order)
      const int l = __ffsll((long long)m) - 1;
      if (readlane_at(qc, l) == lane && lane < C) Mr -= readlane_at(qd, l);
    }
    double lo_r, hi_r, lo_p, hi_p;
    const double mr = wave_tiles(Mr, lo_r, hi_r);
    const double mp = wave_tiles(Mp, lo_p, hi_p);
    const bool use_r = resid && mr > 0.0;
    const double thr = (double)uf * (use_r ? mr : mp);
    const double clo = use_r ? lo_r : lo_p, chi = use_r ? hi_r : hi_p;
    const double cmass = use_r ? Mr : Mp;
    uint64_t hit = __ballot(lane < C && cmass > 0.0 && clo <= thr && thr < chi);
    if (!hit) {  // rounding left the threshold at the end: the last chunk with mass
      const uint64_t pos = __ballot(lane < C && cmass > 0.0);
      hit = pos ? 1ull << (63 - __clzll((long long)pos)) : 0ull;
    }
    const int cstar = hit ? __ffsll((long long)hit) - 1 : -1;
    const uint64_t qm = __ballot(qc >= 0 && qc == cstar);
    if (tid == 0) {
      sh.chunk = cstar;
      sh.thr = thr;
      sh.use_r = use_r ? 1 : 0;
      sh.qmask = qm;
    }
    if (cstar >= 0 && lane == cstar) {
      sh.chunk_lo = clo;
      sh.tieq = tie_prefix;
    }
  }
  __syncthreads();
}

// Dense draw, second part: the planned chunk in id order -- per-thread masses, the thread whose
// mass holds the threshold, then its ids, walked by wave 0 from an LDS copy of that thread's
// span (at most two rounds of 64 lanes).  The span's history hits are penalised in place first
// (hv / hm: WHITV LDS slots per wave), so the per-value work is branch-free: the kept test
// compares values (key order is value order, -0 with +0) and each vector's weights are summed
// in float before the double total.  Returns the token (every thread).
// PRE: the planned chunk's span is already loaded into `sp` (else loaded here).
template <int DT, bool ALIGNED, int NT, bool PRE = false>
__device__ __forceinline__ int64_t dense_pick(const KParams& P, int b, const char* rowp, const RowSum& rs, float T,
                                              float pres, float rep, DrawShared& sh, Span<DT, NT>& sp, uint4* hv,
                                              uint32_t* hm) {
  constexpr int NW = NT / WAVE;
  constexpr int n = Elems<DT>::n, CHE = Elems<DT>::chunk, FE = Span<DT, NT>::FE, SV = Span<DT, NT>::SV;
  static_assert(FE <= 2 * WAVE && SV <= CV_MAX && 64 % n == 0, "a span is walked in two rounds of a wave");
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const bool hist = rs.mode == M_HIST;
  const BonusP bp = bonus_p<DT>(rs, T);
  const double P_cut = hist ? (double)bp(value_of_key<DT>(rs.vcut)) : 0.0;
  if (tid == 0) {
    sh.bonus = V - 1;
    sh.pick_thread = -1;
  }
  __syncthreads();
  const int cstar = sh.chunk;
  if (cstar < 0) return V - 1;
  if constexpr (!PRE) span_load<DT, ALIGNED, NT>(P, b, rowp, cstar, sp);
  if (P.pbits) {
    uint32_t bits[SV];
#pragma unroll
    for (int u = 0; u < SV; ++u)
      bits[u] = (uint32_t)((u * n < 64 ? sp.blo >> (u * n) : sp.bhi >> (u * n - 64)) & ((1ull << n) - 1ull));
    const int wid = tid / WAVE;
    penalize_hits<DT, SV>(sp.v, bits, pres, rep, hv + wid * WHITV, hm + wid * WHITV);
  }
  const bool use_r = sh.use_r != 0;
  const int64_t jlo = (int64_t)cstar * CHE + (int64_t)tid * FE;
  // kept: value > vc; at the cut: value == vc (the cut key's value; -inf without a cut, where
  // values past the row, -inf, weigh exp2(-inf) = 0 and count no tie)
  const float vc = hist ? value_of_key<DT>(rs.vcut) : -INFINITY;
  double mt = 0.0;
  int32_t tt = 0;  // the span's values at the cut key
  float su_prev = 0.f;
#pragma unroll
  for (int u = 0; u < SV; ++u) {
    float su = 0.f;
    // one vector's exponentials at a time, after the previous vector's sum: no weights held
    reg_fence1(sp.v[u], su_prev);
#pragma unroll
    for (int e = 0; e < n; ++e) {
      const float x = vec_elem<DT>(sp.v[u], e);
      const float w = bp(x);
      su += (!hist || x > vc) ? w : 0.f;
      tt += (hist && x == vc) ? 1 : 0;
    }
    mt += (double)su;
    su_prev = su;
  }
  int32_t tie_tot = 0;
  const int32_t tbefore = sh.tieq + block_excl_scan<NW>(tt, sh.red_i, &tie_tot);
  int32_t kept_t = 0;
  if (hist) {
    const int64_t room = (int64_t)rs.ktie - tbefore;
    kept_t = room <= 0 ? 0 : (room < tt ? (int32_t)room : tt);
  }
  double w_t = mt + (kept_t > 0 ? (double)kept_t * P_cut : 0.0);
  const uint64_t qm = use_r ? sh.qmask : 0ull;  // the residual's q ids in this chunk
  for (uint64_t m = qm; m; m &= m - 1ull) {
    const int l = __ffsll((long long)m) - 1;
    if (sh.qid[l] >= jlo && sh.qid[l] < jlo + FE) w_t -= sh.qd[l];
  }
  double tlo, thi;
  block_tiles<NW>(w_t, sh.red_d, tlo, thi);
  const double base = sh.chunk_lo, thr = sh.thr;
  if (w_t > 0.0 && base + tlo <= thr && thr < base + thi) sh.pick_thread = tid;
  __syncthreads();
  int pt = sh.pick_thread;
  if (pt < 0) {
    // rounding left the threshold past this chunk's recomputed mass: the last thread with mass
    const uint64_t lp = block_max_u64<NW>(w_t > 0.0 ? (uint64_t)tid + 1 : 0ull, sh.red_u);
    pt = lp ? (int)lp - 1 : -1;
  }
  if (tid == pt) {  // the span (penalised), for the wave that walks it
#pragma unroll
    for (int u = 0; u < SV; ++u) sh.pv[u] = sp.v[u];
    sh.ptb = tbefore;
    sh.pick_lo = base + tlo;
  }
  __syncthreads();
  if (pt >= 0 && tid < WAVE) {
    // one id a lane in id order: kept cut-key values in rank order, the residual at the q ids,
    // then the running sum from the span's start
    const int lane = tid;
    const int64_t plo = (int64_t)cstar * CHE + (int64_t)pt * FE;
    double run = sh.pick_lo;
    int32_t seen = sh.ptb;  // cut-key values before this round
    int64_t pick = -1, last = -1;
#pragma unroll
    for (int h = 0; h < (FE + WAVE - 1) / WAVE; ++h) {
      const int i = h * WAVE + lane;
      const bool live = i < FE;
      float x = -INFINITY;
      if (live) {
        if constexpr (DT == DSV_BF16)
          x = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(sh.pv)[i]);
        else
          x = reinterpret_cast<const float*>(sh.pv)[i];
      }
      const bool at_cut = live && hist && x == vc;
      const uint64_t cutm = __ballot(at_cut);
      double Pj = 0.0;
      if (at_cut)
        Pj = (int64_t)seen + __popcll(cutm & ((1ull << lane) - 1ull)) < (int64_t)rs.ktie ? P_cut : 0.0;
      else if (live && (!hist || x > vc))
        Pj = (double)bp(x);
      seen += __popcll(cutm);
      const int64_t j = plo + i;
      for (uint64_t m = live ? qm : 0ull; m; m &= m - 1ull) {
        const int l = __ffsll((long long)m) - 1;
        if (sh.qid[l] == j) Pj = fmax(Pj - (double)sh.qv[l], 0.0);
      }
      double wlo, whi;
      const double tot = wave_tiles(Pj, wlo, whi);
      const uint64_t hitj = __ballot(live && Pj > 0.0 && run + whi > thr);
      const uint64_t pos = __ballot(live && Pj > 0.0);
      if (pick < 0 && hitj) pick = plo + h * WAVE + (__ffsll((long long)hitj) - 1);
      if (pos) last = plo + h * WAVE + (63 - __clzll((long long)pos));
      run += tot;
    }
    if (pick < 0) pick = last;  // rounding: the last id with mass
    if (lane == 0 && pick >= 0) sh.bonus = pick;
  }
  __syncthreads();
  return sh.bonus;
}

// ---------------------------------------------------------------------------------------
// Row merge (the last chunk workgroup of a row): chunk partials -> RowSum, support list and
// the step decision.  Rank selection of the row's top-K uses the whole workgroup; the rest
// runs on wave 0.
// ---------------------------------------------------------------------------------------
// A row's merge result in LDS; k_merge's last step stores it (global stores issued earlier
// would hold up every later wait on the vector memory counter).
struct RowOut {
  RowSum rs;
  int32_t ok;   // the step decision
  int32_t nuc;  // 1: listed for the full-histogram pass
};

struct MergeShared {
  uint64_t buf[NCHK * DSV_LIST_K];
  uint64_t top[DSV_LIST_K];
  uint64_t cmin[NCHK];  // each chunk's smallest candidate
  int32_t off[NCHK + 1];
};

template <int DT>
__device__ __forceinline__ void merge_row(const KParams& P, int64_t r, int b, int s, int mode, float T, MergeShared& ms,
                                          DrawShared& ds, const RowPre& pre, RowOut* ro) {
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int C = P.C;
  const ChunkStat* cs = pre.cs;
  int kk = 0;
  if (mode == M_LIST) {
    // (sparse joint rows rank the capacity + 1 largest, whatever their top-k <= capacity)
    const int K = a.sparse_joint ? SJ_CAP + 1 : (pre.top_k < 1 ? 1 : pre.top_k);
    if (tid == 0) {
      int o = 0;
      for (int c = 0; c < C; ++c) {
        ms.off[c] = o;
        o += cs[c].ncand;
      }
      ms.off[C] = o;
    }
    if (tid < C) ms.cmin[tid] = ~0ull;
    // every chunk's candidate slots, loaded together (in-bounds addresses, unused slots dropped)
    const int kc = P.kcand, nslot = C * kc;
    const uint64_t* src = P.cand + r * (int64_t)nslot;
    constexpr int CU = 4;
    for (int base = 0; base < nslot; base += CT * CU) {
      uint64_t v[CU];
#pragma unroll
      for (int u = 0; u < CU; ++u) {
        const int idx = base + u * CT + tid;
        v[u] = src[idx < nslot ? idx : nslot - 1];
      }
      if (base == 0) __syncthreads();  // ms.off
#pragma unroll
      for (int u = 0; u < CU; ++u) {
        const int idx = base + u * CT + tid;
        if (idx < nslot) {
          const int c = idx / kc, i = idx - c * kc;
          if (i < ms.off[c + 1] - ms.off[c]) {
            ms.buf[ms.off[c] + i] = v[u];
            atomicMin(&ms.cmin[c], (unsigned long long)v[u]);
          }
        }
      }
    }
    __syncthreads();
    const int n_all = ms.off[C];
    // A chunk whose list holds K candidates holds its K largest values, so the row's K largest
    // are at or above that list's smallest: the largest such minimum bounds them from below.
    // The candidates at or above it are compacted to the front of the buffer (values are
    // distinct) and ranked among themselves.
    uint64_t lb = 0ull;
    for (int c = 0; c < C; ++c)
      if (ms.off[c + 1] - ms.off[c] >= K && ms.cmin[c] > lb) lb = ms.cmin[c];
    constexpr int PER = NCHK * DSV_LIST_K / CT;
    uint64_t keep_v[PER];
    int nk = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = u * CT + tid;
      keep_v[u] = i < n_all ? ms.buf[i] : 0ull;
      nk += (i < n_all && keep_v[u] >= lb) ? 1 : 0;
    }
    int n_keep = 0;
    int at = block_excl_scan<CT / WAVE>(nk, ds.red_i, &n_keep);  // (its barriers follow every read)
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = u * CT + tid;
      if (i < n_all && keep_v[u] >= lb) ms.buf[at++] = keep_v[u];
    }
    __syncthreads();
    for (int i = tid; i < n_keep; i += CT) {
      const uint64_t v = ms.buf[i];
      int rank = 0;
      for (int j = 0; j < n_keep; ++j) rank += ms.buf[j] > v;
      if (rank < K) ms.top[rank] = v;
    }
    __syncthreads();
    kk = K < n_all ? K : n_all;
  }
  if (tid >= WAVE) return;  // wave 0 finishes the row

  float m_l = -INFINITY;
  int32_t arg_l = INT_MAX;
  double s_l = 0.0;
  if (lane < C) {
    m_l = cs[lane].m;
    arg_l = cs[lane].arg;
    s_l = cs[lane].s;
  }
  // the row max and the first id attaining it (chunks cover increasing ids)
  float M = m_l;
  M = wave_max_f32(M);
  const uint64_t at_max = __ballot(lane < C && m_l == M);
  int32_t arg = readlane_at(arg_l, at_max ? __ffsll((long long)at_max) - 1 : 0);
  if (arg == INT_MAX) arg = 0;  // every value is -inf: the first id
  const int64_t tok = pre.tok;
  RowSum rs;
  rs.mode = mode;
  rs.argmax = arg;
  rs.kmax = key_of<DT>(M);
  rs.vcut = 0u;
  rs.ktie = INT_MAX;
  rs.nlist = 0;
  rs.flags = 0;
  rs.norm = 0;
  rs.S_f = 1.f;
  rs.S_kept = 1.0;
  rs.Z = 1.0;
  rs.m_f = M;
  rs.invZ = 1.f;
  rs.p_draft = 0.f;
  ListEntry* list = P.lists + r * DSV_LIST_K;
  if (mode == M_GREEDY) {
    rs.nlist = 1;
    rs.p_draft = tok == arg ? 1.f : 0.f;
    const int32_t ok = tok >= 0 ? step_accept_lds(ds, a.K, tok, rs.p_draft, pre.u) : 0;
    if (lane == 0) {
      if (!a.candidates) list[0] = ListEntry{arg, 1.f};  // (the step draws from LDS)
      ro->rs = rs;
      ro->ok = ok;
      ro->nuc = 0;
    }
    return;
  }
  const float c2 = log2e_over(T);
  // (support-list rows whose filter does not read Z: p up to the factor 1/Z, renormalised below)
  const bool nz = mode != M_LIST || list_needs_z(a, pre.top_p);
  const double Z =
      nz ? wave_sum(m_l > -INFINITY ? s_l * (double)__builtin_amdgcn_exp2f((m_l - M) * c2) : 0.0) : 1.0;
  const float m_f = M / T;
  const float invZ = (float)(1.0 / Z);
  rs.Z = Z;
  rs.m_f = m_f;
  rs.invZ = invZ;
  // the draft token's adjusted logit (recorded by the chunk that holds it)
  const float xt = (tok >= 0 && tok < a.vocab) ? cs[tok / Elems<DT>::chunk].xtok : -INFINITY;
  if (mode == M_UNF) {
    const float p = (tok >= 0 && tok < a.vocab) ? prob_of(xt, T, m_f, invZ) : 0.f;
    if (a.filter) {  // filtered request with nothing cut: P = p / sum(p)
      rs.norm = 1;
      rs.S_kept = Z * (double)invZ;
      rs.S_f = (float)rs.S_kept;
      rs.p_draft = p / rs.S_f;
    } else {
      rs.p_draft = p;
    }
    // each chunk's mass of P for the bonus draw: its softmax partial sum at the row's scale
    if (lane < C) {
      const double mc = m_l > -INFINITY ? s_l * (double)__builtin_amdgcn_exp2f((m_l - M) * c2) : 0.0;
      ds.cm[lane] = mc * (double)(invZ * (rs.norm ? 1.f / rs.S_f : 1.f));
      ds.ct[lane] = 0;
    }
  } else {
    // LIST: lane j holds the j-th largest candidate
    const bool live = lane < kk;
    const uint64_t pk = live ? ms.top[lane] : 0ull;
    const int32_t id = live ? unpack_id(pk) : INT_MAX;
    const float p = live ? prob_of(value_of_key<DT>(unpack_key(pk)), T, m_f, invZ) : 0.f;
    double lo_p, hi_p;
    const double S_all = wave_tiles((double)p, lo_p, hi_p);
    const float top_p = pre.top_p;
    const float min_p = pre.min_p;
    bool keep;
    if (a.sparse_joint) {
      // The reference's sparse joint target (sampling/sparse/target.py:156-178): of the row's
      // capacity + 1 largest, keep p > 0, p >= p_(k) (every value tied with the k-th) and the
      // nucleus -- the mass of the strictly larger p below top_p, or top_p >= 1.  Equal p are
      // adjacent here, so that mass is the prefix at the first lane holding the lane's p.
      const float p_prev = __shfl(p, lane > 0 ? lane - 1 : 0, WAVE);
      const uint64_t starts = __ballot(live && (lane == 0 || p_prev != p)) | 1ull;
      const uint64_t upto = lane == WAVE - 1 ? ~0ull : (2ull << lane) - 1ull;
      const int first = 63 - __clzll((long long)(starts & upto));
      const double higher = __shfl(lo_p, first, WAVE);
      const int kidx = (pre.top_k < 1 ? 1 : (pre.top_k > kk ? kk : pre.top_k)) - 1;
      const float p_k = readlane_at(p, kidx);
      keep = live && p > 0.f && p >= p_k && (top_p >= 1.f || higher < (double)top_p);
      if (__popcll(__ballot(keep)) > SJ_CAP) {
        // More kept than the packed capacity: the (capacity+1)-th kept value ties the k-th, so
        // the nucleus keeps every p >= p_(k) -- a dense row cut at the k-th key with all of its
        // ties (sparse/target.py:56-76).  Its values at the cut key: those in the chunks' lists
        // (read again: a rare path) and those each list left out (counted by the chunk pass).
        const uint32_t kcut = readlane_at(unpack_key(pk), kidx);
        int32_t nt = 0;
        for (int c = 0; c < C; ++c) {
          const uint64_t* src = P.cand + (r * C + c) * (int64_t)P.kcand;
          const int nc = cs[c].ncand;
          for (int i = lane; i < nc; i += WAVE) nt += unpack_key(src[i]) == kcut;
          if (lane == 0 && unpack_key(ms.cmin[c]) == kcut) nt += cs[c].tieq;
        }
        nt = wave_sum(nt);
        const double S = wave_sum(live && unpack_key(pk) > kcut ? (double)p : 0.0) + (double)nt * (double)p_k;
        rs.mode = M_HIST;
        rs.vcut = kcut;
        rs.ktie = INT_MAX;
        rs.flags = FLAG_SCAN_DRAW;
        rs.S_kept = S;
        rs.S_f = (float)S;
        rs.p_draft = (tok >= 0 && tok < a.vocab && key_of<DT>(xt) >= kcut) ? prob_of(xt, T, m_f, invZ) / rs.S_f : 0.f;
        const int32_t ok = tok >= 0 ? step_accept_lds(ds, a.K, tok, rs.p_draft, pre.u) : 0;
        if (lane == 0) {
          ro->rs = rs;
          ro->ok = ok;
          ro->nuc = 0;
        }
        return;
      }
    } else {
      keep = live && lane < pre.top_k && (!nz || !topp_fails(a.backend, lo_p, p, top_p));
      if (a.need_min_p) {
        if (a.backend == DSV_BACKEND_FLASHINFER) {
          // sequential branch: renormalise over the top-k, top-p on that mass, then min-p
          double lo_a, hi_a;
          wave_tiles(live ? (double)p / S_all : 0.0, lo_a, hi_a);
          keep = live && lane < pre.top_k && lo_a <= (double)top_p;
        }
        const float thr = readlane<0>(p) * min_p;
        if (p < thr) keep = false;
      }
    }
    const double Sk = wave_sum(keep ? (double)p : 0.0);
    const float S_f = (float)Sk;
    rs.S_kept = Sk;
    rs.S_f = S_f;
    const float Pj = p / S_f;
    const uint64_t at_tok = __ballot(keep && (int64_t)id == tok);
    rs.p_draft = at_tok ? readlane_at(Pj, __ffsll((long long)at_tok) - 1) : 0.f;
    // the kept support, sorted by id
    const int32_t kid = keep ? id : INT_MAX;
    int rank = 0;
    for (int i = 0; i < kk; ++i) rank += readlane_at(kid, i) < kid;
    if (keep) {
      if (!a.candidates) list[rank] = ListEntry{id, Pj};
      ds.lst[rank] = ListEntry{id, Pj};
    }
    rs.nlist = __popcll(__ballot(keep));
    if (lane == 0) ds.nlist = rs.nlist;
  }
  const int32_t ok = tok >= 0 ? step_accept_lds(ds, a.K, tok, rs.p_draft, pre.u) : 0;
  if (lane == 0) {
    ro->rs = rs;
    ro->ok = ok;
    ro->nuc = 0;
  }
}

// ---------------------------------------------------------------------------------------
// Nucleus rows (a top-p / min-p cut with top-k > 64).
//
// The chunk pass counts, per chunk, the values whose key lies in a window [wlo, kmax] below the
// chunk max, where wlo is the lowest key whose probability estimate (the chunk's values other than
// its maximum standing for each other chunk's mass) reaches 2 (1 - top_p) / V; the estimate is a
// heuristic, the merge checks what the windows cover.  The row merge knows Z and the exact floor
// eps = (sum p - top_p - 1e-6) / V:
// the values with p < eps hold less than sum p - top_p together, so the cut -- the first value
// in (value desc, id asc) order that top-k, min-p or top-p removes -- is at or above the first
// value below the lowest key kb with p(kb) >= eps.  When every chunk window reaches down to kb
// the merged window counts decide the cut exactly; otherwise the row takes the full-histogram
// path (k_nuc).
// ---------------------------------------------------------------------------------------
constexpr int HC_KEYS = 512;  // merged keys whose per-chunk counts stay in LDS (rows of <= 8 chunks)
struct NucMergeShared {
  uint32_t h[HWIN];  // merged counts, position q = kmax - key
  uint16_t hc[8 * HC_KEYS];  // per-chunk counts at position q (chunk c at c * HC_KEYS + q)
  uint32_t cw[NCHK], ck[NCHK];
  double wm[CT / WAVE];
  int64_t wc[CT / WAVE];
  uint64_t cut[CT / WAVE];
  double cutS[CT / WAVE];
  uint64_t u[CT / WAVE];
  int32_t red_i[CT / WAVE];
  uint32_t kb_row;
  float xtok;
};

// p of a nucleus row at its draft token and the step decision; RowSum out (wave 0).
template <int DT>
__device__ __forceinline__ void nucleus_finish(const KParams& P, int64_t r, int b, int s, RowSum rs, float T,
                                               float xtok, int64_t tok, int64_t tie_tok, RowOut* ro,
                                               const DrawShared* fq = nullptr, float coin = 0.f) {
  const bool kept = key_of<DT>(xtok) > rs.vcut || (key_of<DT>(xtok) == rs.vcut && tie_tok < (int64_t)rs.ktie);
  rs.p_draft = (tok >= 0 && tok < P.a.vocab && kept) ? prob_of(xtok, T, rs.m_f, rs.invZ) / rs.S_f : 0.f;
  int32_t ok = 0;
  if (tok >= 0) ok = fq ? step_accept_lds(*fq, P.a.K, tok, rs.p_draft, coin) : step_accept_wave(P.a, b, s, tok, rs.p_draft);
  if (threadIdx.x == 0) {
    if (ro) {
      ro->rs = rs;
      ro->ok = ok;
      ro->nuc = 0;
    } else {
      P.rowsum[r] = rs;
      P.step_ok[r] = ok;
    }
  }
}

template <int DT>
__device__ __forceinline__ void merge_nucleus(const KParams& P, int64_t r, int b, int s, float T, NucMergeShared& sh,
                                              DrawShared& ds, const RowPre& pre, RowOut* ro) {
  constexpr int NW = CT / WAVE;
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
  const int C = P.C;
  const ChunkStat* cs = pre.cs;
  float m_l = -INFINITY;
  int32_t arg_l = INT_MAX;
  double s_l = 0.0;
  uint32_t w_l = WIN_EMPTY, x_l = 0;
  if (lane < C) {
    m_l = cs[lane].m;
    arg_l = cs[lane].arg;
    s_l = cs[lane].s;
    w_l = cs[lane].wlo;
    x_l = cs[lane].kx;
  }
  float M = m_l;
  M = wave_max_f32(M);
  const uint64_t at_max = __ballot(lane < C && m_l == M);
  int32_t arg = readlane_at(arg_l, at_max ? __ffsll((long long)at_max) - 1 : 0);
  if (arg == INT_MAX) arg = 0;
  const float c2 = log2e_over(T);
  const double Z = wave_sum(m_l > -INFINITY ? s_l * (double)__builtin_amdgcn_exp2f((m_l - M) * c2) : 0.0);
  const float m_f = M / T;
  const float invZ = (float)(1.0 / Z);
  const uint32_t kmax = key_of<DT>(M);
  uint32_t kcov = (lane < C && w_l != WIN_EMPTY) ? w_l : 0u;  // every chunk counted each key >= kcov
  kcov = wave_max_u32(kcov);
  if (tid < C) {
    sh.cw[tid] = w_l;
    sh.ck[tid] = w_l != WIN_EMPTY ? key_of<DT>(m_l) : 0u;
  }
  const float top_p = pre.top_p;
  const float min_p = a.need_min_p ? pre.min_p : 0.f;
  const int topk = pre.top_k;
  const int64_t tok = pre.tok;
  if (tid < WAVE) {
    const double eps = (Z * (double)invZ - (double)top_p - 1e-6) / (double)a.vocab;
    uint32_t kb = 0x80u;  // the lowest finite key: no floor
    if (eps > 0.0 && kmax >= 0x80u) {  // smallest key with p >= eps (p is non-decreasing in the key)
      // the closed form's key, x = T (m_f + ln(eps Z)), as the search's guess
      const float lnp = (__builtin_amdgcn_logf((float)eps) - __builtin_amdgcn_logf(invZ)) * 0.693147180559945309f;
      const uint32_t guess = key_of<DT>(T * (m_f + lnp));
      kb = wave_first_key_near(0x80u, kmax, guess, [&](uint32_t k) {
        return (double)prob_of(value_of_key<DT>(k), T, m_f, invZ) >= eps;
      });
    }
    if (lane == 0) {
      sh.kb_row = kb;
      sh.xtok = (tok >= 0 && tok < a.vocab) ? cs[tok / Elems<DT>::chunk].xtok : -INFINITY;
    }
  }
  __syncthreads();
  RowSum rs;
  rs.mode = M_HIST;
  rs.argmax = arg;
  rs.kmax = kmax;
  rs.vcut = 0u;
  rs.ktie = INT_MAX;
  rs.nlist = 0;
  rs.flags = 0;
  rs.norm = 0;
  rs.m_f = m_f;
  rs.invZ = invZ;
  rs.Z = Z;
  rs.S_kept = 1.0;
  rs.S_f = 1.f;
  rs.p_draft = 0.f;
  if (kmax < 0x80u) {  // no finite value
    if (tid == 0) {
      rs.flags = FLAG_FULL_HIST;
      ro->rs = rs;
      ro->ok = 0;
      ro->nuc = 1;
    }
    return;
  }
  // Every chunk counted each key >= kcov, so a cut found at or above kcov is exact.  The cut
  // is also at or above the first value below the floor kb: only keys >= max(kb, kcov) are
  // scanned (the first value below kb, if the scan keeps every value, is found separately).
  const uint32_t kscan = sh.kb_row > kcov ? sh.kb_row : kcov;
  const int W = (int)(kmax - kscan) + 1;  // <= HWIN: the max's own chunk window ends at kmax
  const bool keep_hc = W <= HC_KEYS && C <= 8;  // the per-chunk counts serve the bonus masses too
  // With the window in the per-chunk tables, the counts' unused tail holds each key's exp terms,
  // computed once: e^(x/T - m_f) (p = that * invZ, as prob_of) and 2^(x c2 - M c2) (the bonus
  // draw's P = that * scale, as BonusP) -- the same floats as the direct formulas.
  float* const ptab = reinterpret_cast<float*>(sh.h + HC_KEYS);
  float* const etab = reinterpret_cast<float*>(sh.h + 2 * HC_KEYS);
  static_assert(3 * HC_KEYS <= HWIN, "exp tables in the counts' tail");
  const float c2b = log2e_over(T), mc2b = value_of_key<DT>(kmax) * c2b;
  for (int q = tid; q < W; q += CT) {
    const uint32_t k = kmax - (uint32_t)q;
    if (keep_hc) {
      const float x = value_of_key<DT>(k);
      ptab[q] = expf(x / T - m_f);
      etab[q] = __builtin_amdgcn_exp2f(fmaf(x, c2b, -mc2b));
    }
    uint32_t cnt = 0;
    for (int c0 = 0; c0 < C; c0 += 8) {  // eight chunks' words loaded together (in-bounds addresses)
      uint32_t word[8], o[8];
      bool in[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u;
        const uint32_t wl = c < C ? sh.cw[c] : WIN_EMPTY;
        in[u] = wl != WIN_EMPTY && k >= wl && k <= sh.ck[c < C ? c : 0];
        o[u] = in[u] ? k - wl : 0u;
        word[u] = P.hpart[(r * C + (c < C ? c : 0)) * (int64_t)(HWIN / 2) + (o[u] >> 1)];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t cu = in[u] ? (word[u] >> ((o[u] & 1u) * 16u)) & 0xFFFFu : 0u;
        cnt += cu;
        if (keep_hc && c0 == 0) sh.hc[u * HC_KEYS + q] = (uint16_t)cu;
      }
    }
    sh.h[q] = cnt;
  }
  __syncthreads();
  // descending scan: wave w owns positions [w*SL, (w+1)*SL)
  const int SL = ((W + NW * WAVE - 1) / (NW * WAVE)) * WAVE;
  const int q_end = (wid + 1) * SL < W ? (wid + 1) * SL : W;
  const float thr_minp = prob_of(M, T, m_f, invZ) * min_p;
  double mt = 0.0;
  int64_t cw = 0;
  for (int q = wid * SL + lane; q < q_end; q += WAVE) {
    const uint32_t cnt = sh.h[q];
    if (!cnt) continue;
    const float p = keep_hc ? ptab[q] * invZ : prob_of(value_of_key<DT>(kmax - (uint32_t)q), T, m_f, invZ);
    mt += (double)cnt * (double)p;
    cw += cnt;
  }
  mt = wave_sum(mt);
  cw = wave_sum(cw);
  if (lane == 0) {
    sh.wm[wid] = mt;
    sh.wc[wid] = cw;
  }
  __syncthreads();
  double run_S = 0.0, m_total = 0.0;
  int64_t run_C = 0;
  for (int i = 0; i < NW; ++i) {
    if (i < wid) {
      run_S += sh.wm[i];
      run_C += sh.wc[i];
    }
    m_total += sh.wm[i];
  }
  // The first value (value desc, id asc) that the filter (rank < tk, p >= mp * max, mass
  // ahead within tp) removes in the merged window: fc = its key | tie index << 32 (~0: none in
  // the window), fS the mass kept before it.
  auto find_cut = [&](int tk, float mp, float tp, uint64_t& fc, double& fS) {
    double rS = run_S;
    int64_t rC = run_C;
    uint64_t cut = ~0ull;
    double cutS = 0.0;
    for (int q0 = wid * SL; q0 < q_end && cut == ~0ull; q0 += WAVE) {
      const int q = q0 + lane;
      const uint32_t cnt = q < q_end ? sh.h[q] : 0u;
      if (__ballot(cnt != 0u) == 0ull) continue;
      const uint32_t k = kmax - (uint32_t)q;
      const float p = !cnt ? 0.f : keep_hc ? ptab[q] * invZ : prob_of(value_of_key<DT>(k), T, m_f, invZ);
      double lo_m, hi_m;
      const double it_m = wave_tiles((double)cnt * (double)p, lo_m, hi_m);
      int64_t c_excl = wave_incl_scan((int64_t)cnt);
      const int64_t it_c = readlane<WAVE - 1>(c_excl);
      c_excl -= cnt;
      uint64_t f = ~0ull;
      double fSl = 0.0;
      if (cnt) {
        const double sb = rS + lo_m;
        const int64_t fail = cut_index(a.backend, cnt, p, sb, rC + c_excl, tk, mp, thr_minp, tp);
        if (fail < (int64_t)cnt) {
          f = ((uint64_t)(uint32_t)fail << 32) | k;
          fSl = sb + (double)fail * (double)p;
        }
      }
      const uint64_t who = __ballot(f != ~0ull);
      if (who) {
        const int src = __ffsll((long long)who) - 1;
        cut = readlane_at(f, src);
        cutS = readlane_at(fSl, src);
      }
      rS += it_m;
      rC += it_c;
    }
    __syncthreads();  // (readers of an earlier call's results)
    if (lane == 0) {
      sh.cut[wid] = cut;
      sh.cutS[wid] = cutS;
    }
    __syncthreads();
    fc = ~0ull;
    fS = 0.0;
    for (int i = 0; i < NW && fc == ~0ull; ++i) {
      fc = sh.cut[i];
      fS = sh.cutS[i];
    }
  };
  const bool x_untracked = __ballot(lane < C && x_l == KX_UNKNOWN) != 0ull;
  float top_p_eff = top_p;
  if (a.backend == DSV_BACKEND_FLASHINFER && min_p > 0.f) {
    // flashinfer's min-p branch renormalises over the top-k before its top-p test: a value is
    // kept while (mass ahead) / S_k <= top_p, S_k the top-k's mass (a rank-only cut first)
    uint64_t kc;
    double kS;
    find_cut(topk, 0.f, INFINITY, kc, kS);
    if (kc == ~0ull && (int64_t)topk < a.vocab) {
      // the top-k reaches below the window: the full histogram decides the row
      if (tid == 0) {
        rs.flags = FLAG_FULL_HIST;
        ro->rs = rs;
        ro->ok = 0;
        ro->nuc = 1;
      }
      return;
    }
    top_p_eff = (float)((double)top_p * (kc != ~0ull ? kS : Z * (double)invZ));
  }
  uint64_t fc;
  double fS;
  find_cut(topk, min_p, top_p_eff, fc, fS);
  // No value at or above kscan is removed.  When their mass (all of it counted: each chunk
  // counted every key >= kcov) already exceeds the top-p bound by more than the probabilities'
  // rounding, every value below kscan has at least that mass ahead and is removed as well: the
  // cut sits just below kscan, whatever values lie there (peaked rows, whose nucleus is a few
  // tokens far above the other chunks' windows).
  const bool cut_below = fc == ~0ull && m_total > (double)top_p_eff + 1e-5;
  if (fc == ~0ull && !cut_below && (kcov > sh.kb_row || x_untracked)) {
    // the cut lies below a chunk's window (or below every window, where a chunk did not
    // track its largest value): the full histogram decides it
    if (tid == 0) {
      rs.flags = FLAG_FULL_HIST;
      ro->rs = rs;
      ro->ok = 0;
      ro->nuc = 1;
    }
    return;
  }
  if (fc != ~0ull) {
    rs.vcut = (uint32_t)fc;
    rs.ktie = (int32_t)(fc >> 32);
    rs.S_kept = fS;
  } else if (cut_below) {
    rs.vcut = kscan - 1u;  // (kscan >= 0x80, the lowest finite key)
    rs.ktie = 0;
    rs.S_kept = m_total;
  } else {
    // every value at or above kscan is kept: the cut is the first value below kscan (tie 0)
    uint64_t below = 0;
    for (int c = 0; c < C; ++c) {
      const uint32_t wl = sh.cw[c];
      if (wl == WIN_EMPTY) continue;
      const uint32_t kh = sh.ck[c] < kscan ? sh.ck[c] : kscan - 1u;
      for (uint32_t k = wl + (uint32_t)tid; wl <= kh && k <= kh; k += CT) {
        const uint32_t o = k - wl;
        const uint32_t word = P.hpart[(r * C + c) * (int64_t)(HWIN / 2) + (o >> 1)];
        if ((word >> ((o & 1u) * 16u)) & 0xFFFFu) below = below > k ? below : k;
      }
    }
    if (lane < C) below = below > x_l ? below : x_l;
    below = block_max_u64<NW>(below, sh.u);
    rs.vcut = (uint32_t)below;
    rs.ktie = below ? 0 : INT_MAX;
    rs.S_kept = m_total;
  }
  rs.S_f = (float)rs.S_kept;
  // For the bonus draw: each chunk's mass of P over the keys above the cut, and its count of
  // values at the cut key.  Every key above the cut is in every window (the cut is at or above
  // kcov, or below every counted value), so the window counts hold them all.
  const BonusP bp = bonus_p<DT>(rs, T);
  if (keep_hc && fc != ~0ull) {
    // the cut is in the merged window: every key above it, and the cut key, are in the LDS
    // counts.  Wave w takes chunks w and w + NW (C <= 8) in one pass over the keys.
    static_assert(2 * NW >= 8, "two chunks a wave cover the per-chunk tables");
    const int c2w[2] = {wid, wid + NW};
    double mc[2] = {0.0, 0.0};
    int32_t tc[2] = {0, 0};
    for (int q = lane; q < W; q += WAVE) {
      const uint32_t k = kmax - (uint32_t)q;
      const float e = etab[q] * bp.scale;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t cnt = c2w[h] < C ? sh.hc[c2w[h] * HC_KEYS + q] : 0u;
        if (k > rs.vcut && cnt) mc[h] += (double)cnt * (double)e;
        if (k == rs.vcut) tc[h] = (int32_t)cnt;
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mc[h] = wave_sum(mc[h]);
      tc[h] = wave_sum(tc[h]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c2w[h];
      if (lane == 0 && c < C) {
        ds.cm[c] = mc[h];
        ds.ct[c] = tc[h];
        if (!a.candidates) P.rties[r * NCHK + c] = tc[h];  // (for k_dense_p; the step keeps them in LDS)
      }
    }
  } else {
  for (int c = wid; c < C; c += NW) {
    const uint32_t wl = sh.cw[c], kh = sh.ck[c];
    double mc = 0.0;
    int32_t tc = 0;
    if (wl != WIN_EMPTY) {
      const uint32_t k0 = rs.vcut + 1u > wl ? rs.vcut + 1u : wl;
      const uint32_t* hp = P.hpart + (r * C + c) * (int64_t)(HWIN / 2);
      for (uint32_t k1 = k0 + (uint32_t)lane; k1 <= kh; k1 += 4 * WAVE) {  // four keys a lane together
        uint32_t word[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t k = k1 + (uint32_t)(u * WAVE);
          word[u] = hp[(k <= kh ? k - wl : 0u) >> 1];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t k = k1 + (uint32_t)(u * WAVE);
          const uint32_t cnt = k <= kh ? (word[u] >> (((k - wl) & 1u) * 16u)) & 0xFFFFu : 0u;
          if (cnt) mc += (double)cnt * (double)bp(value_of_key<DT>(k));
        }
      }
      if (lane == 0 && rs.vcut >= wl && rs.vcut <= kh) {
        const uint32_t o = rs.vcut - wl;
        tc = (int32_t)((hp[o >> 1] >> ((o & 1u) * 16u)) & 0xFFFFu);
      }
    }
    mc = wave_sum(mc);
    if (lane == 0) {
      ds.cm[c] = mc;
      ds.ct[c] = tc;
      if (!a.candidates) P.rties[r * NCHK + c] = tc;
    }
  }
  }
  const float xt = sh.xtok;
  if (tid < WAVE) {
    // values of the draft token's key ahead of it: the whole counts of the chunks before its
    // chunk (the key is in every window when it is the cut key) and its chunk's own count
    int64_t tie_tok = 0;
    const uint32_t kt = key_of<DT>(xt);
    if (tok >= 0 && kt == rs.vcut && rs.ktie > 0 && rs.ktie != INT_MAX && lane < C) {
      constexpr int64_t CHE = Elems<DT>::chunk;
      const int64_t c_lo = (int64_t)lane * CHE, c_hi = c_lo + CHE;
      if (c_hi <= tok) {
        const uint32_t wl = sh.cw[lane];
        if (wl != WIN_EMPTY && kt >= wl && kt <= sh.ck[lane]) {
          const uint32_t o = kt - wl;
          const uint32_t word = P.hpart[(r * C + lane) * (int64_t)(HWIN / 2) + (o >> 1)];
          tie_tok = (word >> ((o & 1u) * 16u)) & 0xFFFFu;
        }
      } else if (c_lo <= tok) {
        tie_tok = cs[lane].tieq;
      }
    }
    tie_tok = wave_sum(tie_tok);
    nucleus_finish<DT>(P, r, b, s, rs, T, xt, tok, tie_tok, ro, &ds, pre.u);
  }
}

// ---------------------------------------------------------------------------------------
// k_nuc: nucleus rows whose windows fall short -- the full 65536-key value histogram, built in
// LDS slices of at most NUC_SLICE values (16-bit counters cannot wrap) and accumulated in
// registers; one workgroup per row, persistent over the rows.
// ---------------------------------------------------------------------------------------
constexpr int NUC_GRID = 64;  // k_nuc workgroups (persistent over the full-histogram rows)
constexpr int NUC_GRID_F32 = 256;  // k_nuc workgroups over float32 rows (LDS only: one a CU)
constexpr int NUC_WAVES = NUC_THREADS / WAVE;
constexpr int NUC_WPW = HIST_WORDS / NUC_WAVES;  // histogram words per wave
constexpr int NUC_ITERS = NUC_WPW / WAVE;        // words per lane

struct NucShared {
  double d[NUC_WAVES];
  double wm[NUC_WAVES];
  int64_t wc[NUC_WAVES];
  uint64_t cut[NUC_WAVES];  // (tie << 32 | key) of each wave's first cut key, ~0 if none
  double cutS[NUC_WAVES];
  float xtok;
  uint32_t ktok;
};

// Word wd of the histogram holds the 16-bit counts of keys 2wd (low half) and 2wd+1 (high).
// Wave w owns words HIST_WORDS-1-w*NUC_WPW-64*i-lane for i = 0, 1, ...: consecutive lanes read
// consecutive words (no bank conflicts) and each wave's slice runs in descending key order.
__device__ __forceinline__ int nuc_word(int wid, int i, int lane) {
  return HIST_WORDS - 1 - wid * NUC_WPW - WAVE * i - lane;
}

template <int DT, bool ALIGNED>
// area: the workgroup's 65536-key accumulation area in P.nhist; ro: the row's result into LDS
// (nullptr: RowSum and step decision stored to their arrays).
__device__ __forceinline__ void nuc_row(const KParams& P, int64_t r, uint32_t* hist, NucShared& sh, int area,
                                        RowOut* ro) {
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
  int b = 0, s = 0;
  row_request(a, r, b, s);
  RowSum rs = P.rowsum[r];
  const int64_t V = a.vocab;
  const char* rowp = row_ptr(a, r);
  const float T = a.temperatures[b];
  const int topk = a.top_ks[b];
  const bool pen = P.pbits != nullptr;
  const float pres = pen && a.presence ? a.presence[b] : 0.f;
  const float rep = pen && a.repetition ? a.repetition[b] : 1.f;
  const int64_t tok = step_token(a, b, s);
  if (tid == 0) {
    float xt = -INFINITY;
    if (tok >= 0 && tok < V) {
      xt = load_elem<DT>(rowp, tok);
      if (pen && pen_test(P, b, tok)) xt = penalize<DT>(xt, pres, rep);
    }
    sh.xtok = xt;
    sh.ktok = key_of<DT>(xt);
  }
  __syncthreads();
  const uint32_t ktok = sh.ktok;
  // 32-bit counts of key pairs, this workgroup's own area: (key 2wd, key 2wd + 1) at index wd
  uint2* gsum = reinterpret_cast<uint2*>(P.nhist) + (int64_t)area * HIST_WORDS;
  uint32_t tie_before = 0;
  auto count = [&](float x, int64_t j) {
    const uint32_t k = key_of<DT>(x);
    if (k != NEG_INF_BF16_KEY) {
      atomicAdd(&hist[k >> 1], 1u << ((k & 1u) * 16u));
      tie_before += (k == ktok && j < tok) ? 1u : 0u;
    }
  };
  constexpr int U = 4;
  for (int64_t s0 = 0; s0 < V; s0 += NUC_SLICE) {
    const int64_t s1 = s0 + NUC_SLICE < V ? s0 + NUC_SLICE : V;
    {
      uint4* h4 = reinterpret_cast<uint4*>(hist);
      for (int i = tid; i < HIST_WORDS / 4; i += NUC_THREADS) h4[i] = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const int64_t vb = s0 / 8;                              // NUC_SLICE is a multiple of 8
    const int64_t ve = ALIGNED ? s1 / 8 : (s1 + 7) / 8;     // vectors read whole
    for (int64_t q0 = vb; q0 < ve; q0 += (int64_t)NUC_THREADS * U) {
      uint4 w[U];
      uint32_t bits[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t vi = q0 + (int64_t)u * NUC_THREADS + tid;
        if constexpr (ALIGNED)
          w[u] = load_vec_raw(rowp, vi < ve ? vi : ve - 1);
        else
          w[u] = load_vec<DT>(rowp, vi, s1, false);
        const uint32_t bw = pen ? pen_bits(P, b, (vi < ve ? vi : vb) * 8, 8) : 0u;
        bits[u] = vi < ve ? bw : 0u;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t vi = q0 + (int64_t)u * NUC_THREADS + tid;
        if (vi >= ve) continue;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t j = vi * 8 + e;
          float x = vec_elem<DT>(w[u], e);
          if ((bits[u] >> e) & 1u) x = penalize<DT>(x, pres, rep);
          if (ALIGNED || j < s1) count(x, j);
        }
      }
    }
    if (ALIGNED && tid == 0)
      for (int64_t j = ve * 8; j < s1; ++j) {  // the row's partial last vector
        float x = load_elem<DT>(rowp, j);
        if (pen && pen_test(P, b, j)) x = penalize<DT>(x, pres, rep);
        count(x, j);
      }
    __syncthreads();
    for (int i = 0; i < NUC_ITERS; ++i) {  // each thread owns its words: no atomics
      const int wd = nuc_word(wid, i, lane);
      const uint32_t h = hist[wd];
      uint2 g = s0 ? gsum[wd] : make_uint2(0u, 0u);
      g.x += h & 0xFFFFu;
      g.y += h >> 16;
      gsum[wd] = g;
    }
    __syncthreads();
  }
  const int64_t tie_tok = (int64_t)block_sum<NUC_WAVES>((double)tie_before, sh.d);
  const float m_f = rs.m_f, invZ = rs.invZ;
  const float M = value_of_key<DT>(rs.kmax);
  // mass per wave (descending-key slices), then each wave's starting prefix
  double mt = 0.0;
  int64_t cw = 0;
  for (int i = 0; i < NUC_ITERS; ++i) {
    const int wd = nuc_word(wid, i, lane);
    const uint2 g = gsum[wd];
    if (g.y) {
      mt += (double)g.y * (double)prob_of(value_of_key<DT>(2u * (uint32_t)wd + 1u), T, m_f, invZ);
      cw += g.y;
    }
    if (g.x) {
      mt += (double)g.x * (double)prob_of(value_of_key<DT>(2u * (uint32_t)wd), T, m_f, invZ);
      cw += g.x;
    }
  }
  mt = wave_sum(mt);
  cw = wave_sum(cw);
  if (lane == 0) {
    sh.wm[wid] = mt;
    sh.wc[wid] = cw;
  }
  __syncthreads();
  double run_S = 0.0, m_total = 0.0;
  int64_t run_C = 0;
  for (int i = 0; i < NUC_WAVES; ++i) {
    if (i < wid) {
      run_S += sh.wm[i];
      run_C += sh.wc[i];
    }
    m_total += sh.wm[i];
  }
  const float top_p = a.top_ps[b];
  const float min_p = (a.need_min_p && a.min_ps) ? a.min_ps[b] : 0.f;
  const float thr_minp = prob_of(M, T, m_f, invZ) * min_p;
  // The first value (value desc, id asc) that the filter (rank < tk, p >= mp * max, mass ahead
  // within tp) removes: fc = its key | tie index << 32 (~0: none), fS the mass kept before it.
  auto find_cut = [&](int tk, float mp, float tp, uint64_t& fc, double& fS) {
    double rS = run_S;
    int64_t rC = run_C;
    uint64_t cut = ~0ull;
    double cutS = 0.0;
    for (int i = 0; i < NUC_ITERS && cut == ~0ull; ++i) {
      const int wd = nuc_word(wid, i, lane);
      const uint2 g = gsum[wd];
      const uint32_t c_hi = g.y, c_lo = g.x;
      if (__ballot((c_hi | c_lo) != 0u) == 0ull) continue;
      const uint32_t k_hi = 2u * (uint32_t)wd + 1u, k_lo = 2u * (uint32_t)wd;
      const float p_hi = c_hi ? prob_of(value_of_key<DT>(k_hi), T, m_f, invZ) : 0.f;
      const float p_lo = c_lo ? prob_of(value_of_key<DT>(k_lo), T, m_f, invZ) : 0.f;
      double lo_m, hi_m;
      const double it_m = wave_tiles((double)c_hi * (double)p_hi + (double)c_lo * (double)p_lo, lo_m, hi_m);
      const int64_t c_word = (int64_t)c_hi + c_lo;
      int64_t c_excl = wave_incl_scan(c_word);
      const int64_t it_c = readlane<WAVE - 1>(c_excl);
      c_excl -= c_word;
      uint64_t f = ~0ull;
      double fSl = 0.0;
      double sb = rS + lo_m;
      int64_t cb = rC + c_excl;
      if (c_hi) {
        const int64_t fail = cut_index(a.backend, c_hi, p_hi, sb, cb, tk, mp, thr_minp, tp);
        if (fail < (int64_t)c_hi) {
          f = ((uint64_t)(uint32_t)fail << 32) | k_hi;
          fSl = sb + (double)fail * (double)p_hi;
        } else {
          sb += (double)c_hi * (double)p_hi;
          cb += c_hi;
        }
      }
      if (c_lo && f == ~0ull) {
        const int64_t fail = cut_index(a.backend, c_lo, p_lo, sb, cb, tk, mp, thr_minp, tp);
        if (fail < (int64_t)c_lo) {
          f = ((uint64_t)(uint32_t)fail << 32) | k_lo;
          fSl = sb + (double)fail * (double)p_lo;
        }
      }
      const uint64_t who = __ballot(f != ~0ull);
      if (who) {
        const int src = __ffsll((long long)who) - 1;
        cut = readlane_at(f, src);
        cutS = readlane_at(fSl, src);
      }
      rS += it_m;
      rC += it_c;
    }
    __syncthreads();  // (readers of an earlier call's results)
    if (lane == 0) {
      sh.cut[wid] = cut;
      sh.cutS[wid] = cutS;
    }
    __syncthreads();
    fc = ~0ull;
    fS = 0.0;
    for (int i = 0; i < NUC_WAVES && fc == ~0ull; ++i) {
      fc = sh.cut[i];
      fS = sh.cutS[i];
    }
  };
  float top_p_eff = top_p;
  if (a.backend == DSV_BACKEND_FLASHINFER && min_p > 0.f) {
    // flashinfer's min-p branch: top-p on the mass renormalised over the top-k (S_k from a
    // rank-only cut; no rank cut: the whole mass)
    uint64_t kc;
    double kS;
    find_cut(topk, 0.f, INFINITY, kc, kS);
    top_p_eff = (float)((double)top_p * (kc != ~0ull ? kS : m_total));
  }
  uint64_t fc;
  double fS;
  find_cut(topk, min_p, top_p_eff, fc, fS);
  if (tid < WAVE) {
    if (fc == ~0ull) {
      rs.vcut = 0u;
      rs.ktie = INT_MAX;
      rs.S_kept = m_total;
    } else {
      rs.vcut = (uint32_t)fc;
      rs.ktie = (int32_t)(fc >> 32);
      rs.S_kept = fS;
    }
    rs.S_f = (float)rs.S_kept;
    nucleus_finish<DT>(P, r, b, s, rs, T, sh.xtok, tok, tie_tok, ro);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------
// Float32 nucleus rows: the cut by a radix descent over the 32-bit value keys.  Level 0 bins the
// keys' top 11 bits over the row, level 1 the next 11 bits inside one level-0 bin, level 2 the
// last 10 bits inside one level-1 bin (exact keys).  Level 0 / 1 bins carry value counts and
// masses in fixed point (p scaled by 2^62, integer sums: independent of the order of the
// additions).  The cut test of a key gets stronger as the key falls (more values and mass ahead,
// smaller p), so a bin can hold the cut only when the test holds at its smallest key, which is
// bounded with the bin's lowest possible p; the first such bin (descending), or failing that
// the next non-empty bin, holds the cut.  Each bin searched costs one pass over the row.
// ---------------------------------------------------------------------------------------
constexpr int F32_BINS = 2048, F32_KEYS = 1024;
constexpr double FX_ONE = 4611686018427387904.0;  // 2^62
constexpr uint32_t F32_NEG_INF_KEY = 0x007FFFFFu;  // key of -inf; keys at or below it hold no value
struct F32NucLds {
  uint32_t cnt[2][F32_BINS];
  uint64_t mass[2][F32_BINS];
  uint32_t pcnt[2][F32_BINS];   // values in the bins above (descending bin order)
  uint64_t pmass[2][F32_BINS];  // their mass
  uint32_t cnt3[F32_KEYS];
};
struct F32NucShared {
  uint64_t u[NUC_WAVES], v[NUC_WAVES];
  double d[NUC_WAVES];
  int32_t best;
  uint32_t cut_key;
  int32_t cut_tie;
  double cut_S;
};

// One pass over the row: counts (and, levels 0 and 1, masses) of the values whose key matches the
// level's prefix.  Level 0 also counts the values at the draft token's key before the token.
template <bool ALIGNED>
__device__ __forceinline__ void f32_pass(const KParams& P, int b, const char* rowp, float pres, float rep, float T,
                                         float m_f, float invZ, int level, uint32_t prefix, F32NucLds& L,
                                         uint32_t ktok, int64_t tok, uint32_t& tie_before) {
  const int tid = threadIdx.x;
  const int64_t V = P.a.vocab;
  const bool pen = P.pbits != nullptr;
  uint32_t* cnt = level == 2 ? L.cnt3 : L.cnt[level];
  uint64_t* mass = level == 2 ? nullptr : L.mass[level];
  const int nb = level == 2 ? F32_KEYS : F32_BINS;
  for (int i = tid; i < nb; i += NUC_THREADS) {
    cnt[i] = 0u;
    if (mass) mass[i] = 0ull;
  }
  __syncthreads();
  auto count = [&](float x, int64_t j) {
    const uint32_t k = f32_key(x);
    if (k <= F32_NEG_INF_KEY) return;
    uint32_t bin;
    if (level == 0) {
      bin = k >> 21;
      tie_before += (k == ktok && j < tok) ? 1u : 0u;
    } else if (level == 1) {
      if ((k >> 21) != prefix) return;
      bin = (k >> 10) & (F32_BINS - 1);
    } else {
      if ((k >> 10) != prefix) return;
      bin = k & (F32_KEYS - 1);
    }
    atomicAdd(&cnt[bin], 1u);
    if (mass) atomicAdd((unsigned long long*)&mass[bin], (unsigned long long)((double)prob_of(x, T, m_f, invZ) * FX_ONE));
  };
  constexpr int U = 4;
  const int64_t ve = ALIGNED ? V / 4 : (V + 3) / 4;
  for (int64_t q0 = 0; q0 < ve; q0 += (int64_t)NUC_THREADS * U) {
    uint4 w[U];
    uint32_t bits[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = q0 + (int64_t)u * NUC_THREADS + tid;
      if constexpr (ALIGNED)
        w[u] = load_vec_raw(rowp, vi < ve ? vi : ve - 1);
      else
        w[u] = load_vec<DSV_F32>(rowp, vi, V, false);
      const uint32_t bw = pen ? pen_bits(P, b, (vi < ve ? vi : 0) * 4, 4) : 0u;
      bits[u] = vi < ve ? bw : 0u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = q0 + (int64_t)u * NUC_THREADS + tid;
      if (vi >= ve) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t j = vi * 4 + e;
        float x = vec_elem<DSV_F32>(w[u], e);
        if ((bits[u] >> e) & 1u) x = penalize<DSV_F32>(x, pres, rep);
        if (ALIGNED || j < V) count(x, j);
      }
    }
  }
  if (ALIGNED && tid == 0)
    for (int64_t j = ve * 4; j < V; ++j) {  // the row's partial last vector
      float x = load_elem<DSV_F32>(rowp, j);
      if (pen && pen_test(P, b, j)) x = penalize<DSV_F32>(x, pres, rep);
      count(x, j);
    }
  __syncthreads();
}

// Exclusive prefixes of a level's bins in descending bin order (thread t owns bins 2047 - 4t ..
// 2044 - 4t, highest first).
__device__ __forceinline__ void f32_prefix(F32NucLds& L, int level, F32NucShared& sh) {
  const int tid = threadIdx.x;
  uint64_t c = 0, m = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int bin = F32_BINS - 1 - 4 * tid - e;
    L.pcnt[level][bin] = (uint32_t)c;
    L.pmass[level][bin] = m;
    c += L.cnt[level][bin];
    m += L.mass[level][bin];
  }
  uint64_t tc = 0, tm = 0;
  const uint64_t cb = block_excl_scan<NUC_WAVES>(c, sh.u, &tc);
  const uint64_t mb = block_excl_scan<NUC_WAVES>(m, sh.v, &tm);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int bin = F32_BINS - 1 - 4 * tid - e;
    L.pcnt[level][bin] += (uint32_t)cb;
    L.pmass[level][bin] += mb;
  }
  __syncthreads();
}

// The first non-empty bin of a level after descending rank `after` (rank = 2047 - bin) -- with
// `test`, the first one that can hold the cut given the values and mass ahead of the level
// (base_c, base_m).  Returns the bin, -1 for none.
__device__ __forceinline__ int f32_next(const F32NucLds& L, int level, int after, bool test, uint32_t prefix,
                                        uint64_t base_c, uint64_t base_m, float T, float m_f, float invZ, int backend,
                                        int topk, float min_p, float thr_minp, float top_p, F32NucShared& sh) {
  const int tid = threadIdx.x;
  if (tid == 0) sh.best = INT_MAX;
  __syncthreads();
  int best = INT_MAX;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rank = 4 * tid + e, bin = F32_BINS - 1 - rank;
    const uint32_t cb = L.cnt[level][bin];
    if (rank <= after || cb == 0u || rank >= best) continue;
    bool ok = true;
    if (test) {
      uint32_t klo = level == 0 ? (uint32_t)bin << 21 : (prefix << 21) | ((uint32_t)bin << 10);
      if (klo <= F32_NEG_INF_KEY) klo = F32_NEG_INF_KEY + 1u;
      const float p_lo = prob_of(key_to_f32(klo), T, m_f, invZ);
      const uint64_t n_ge = base_c + L.pcnt[level][bin] + cb;
      const double S_ge = (double)(base_m + L.pmass[level][bin] + L.mass[level][bin]) / FX_ONE;
      ok = (min_p > 0.f && p_lo < thr_minp) || (n_ge - 1 >= (uint64_t)(topk > 0 ? topk : 0)) ||
           topp_fails(backend, S_ge - (double)p_lo, p_lo, top_p);
    }
    if (ok) best = rank;
  }
  if (best != INT_MAX) atomicMin(&sh.best, best);
  __syncthreads();
  const int r = sh.best;
  __syncthreads();
  return r == INT_MAX ? -1 : F32_BINS - 1 - r;
}

// The exact keys of one level-1 bin in descending order: the first key with a failing tie.
// Returns true with the cut in sh (key, tie, mass ahead of the cut).
__device__ __forceinline__ bool f32_walk(const F32NucLds& L, uint32_t prefix, uint64_t base_c, uint64_t base_m,
                                         float T, float m_f, float invZ, int backend, int topk, float min_p,
                                         float thr_minp, float top_p, F32NucShared& sh) {
  const int tid = threadIdx.x;
  uint32_t c[2];
  float pk[2];
  double m = 0.0;
  uint64_t n = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t lo = (uint32_t)(F32_KEYS - 1 - 2 * tid - e);
    c[e] = L.cnt3[lo];
    pk[e] = c[e] ? prob_of(key_to_f32((prefix << 10) | lo), T, m_f, invZ) : 0.f;
    m += (double)c[e] * (double)pk[e];
    n += c[e];
  }
  uint64_t tn = 0;
  double tm = 0.0;
  const uint64_t nb = block_excl_scan<NUC_WAVES>(n, sh.u, &tn);
  const double mb = block_excl_scan<NUC_WAVES>(m, sh.d, &tm);
  if (tid == 0) sh.best = INT_MAX;
  __syncthreads();
  double Sb = (double)base_m / FX_ONE + mb;
  uint64_t Nb = base_c + nb;
  int32_t my_tie = 0;
  uint32_t my_key = 0;
  double my_S = 0.0;
  int my_rank = INT_MAX;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    if (c[e] && my_rank == INT_MAX) {
      const int64_t fail = cut_index(backend, c[e], pk[e], Sb, (int64_t)Nb, topk, min_p, thr_minp, top_p);
      if (fail < (int64_t)c[e]) {
        my_rank = 2 * tid + e;
        my_key = (prefix << 10) | (uint32_t)(F32_KEYS - 1 - my_rank);
        my_tie = (int32_t)fail;
        my_S = Sb + (double)fail * (double)pk[e];
      }
    }
    Sb += (double)c[e] * (double)pk[e];
    Nb += c[e];
  }
  if (my_rank != INT_MAX) atomicMin(&sh.best, my_rank);
  __syncthreads();
  const bool found = sh.best != INT_MAX;
  if (found && my_rank == sh.best) {
    sh.cut_key = my_key;
    sh.cut_tie = my_tie;
    sh.cut_S = my_S;
  }
  __syncthreads();
  return found;
}

template <bool ALIGNED>
__device__ __forceinline__ void nuc_row_f32(const KParams& P, int64_t r, F32NucLds& L, F32NucShared& sh,
                                            RowOut* ro) {
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x;
  int b = 0, s = 0;
  row_request(a, r, b, s);
  RowSum rs = P.rowsum[r];
  const int64_t V = a.vocab;
  const char* rowp = row_ptr(a, r);
  const float T = a.temperatures[b];
  const int topk = a.top_ks[b];
  const bool pen = P.pbits != nullptr;
  const float pres = pen && a.presence ? a.presence[b] : 0.f;
  const float rep = pen && a.repetition ? a.repetition[b] : 1.f;
  const float top_p = a.top_ps[b];
  const float min_p = (a.need_min_p && a.min_ps) ? a.min_ps[b] : 0.f;
  const int64_t tok = step_token(a, b, s);
  float xt = -INFINITY;
  if (tok >= 0 && tok < V) {
    xt = load_elem<DSV_F32>(rowp, tok);
    if (pen && pen_test(P, b, tok)) xt = penalize<DSV_F32>(xt, pres, rep);
  }
  const uint32_t ktok = f32_key(xt);
  const float m_f = rs.m_f, invZ = rs.invZ;
  const float thr_minp = prob_of(key_to_f32(rs.kmax), T, m_f, invZ) * min_p;
  uint32_t tie_before = 0, unused = 0;
  f32_pass<ALIGNED>(P, b, rowp, pres, rep, T, m_f, invZ, 0, 0u, L, ktok, tok, tie_before);
  f32_prefix(L, 0, sh);
  const int64_t tie_tok = (int64_t)block_sum<NUC_WAVES>((uint64_t)tie_before, sh.u);
  // The first value (value desc, id asc) that the filter (rank < tk, p >= mp * max, mass ahead
  // within tp) removes, into sh.cut_key / cut_tie / cut_S; false when it keeps every value.
  // The level-0 bins serve every call.
  auto descend = [&](int tk, float mp, float tp) -> bool {
    bool found = false;
    int b0 = f32_next(L, 0, -1, true, 0u, 0ull, 0ull, T, m_f, invZ, a.backend, tk, mp, thr_minp, tp, sh);
    // the first bin that can hold the cut, else the next non-empty one (a margin of rounding
    // may need one more)
    for (int t0 = 0; t0 < 3 && b0 >= 0 && !found; ++t0) {
      const uint64_t c0 = L.pcnt[0][b0], m0 = L.pmass[0][b0];
      f32_pass<ALIGNED>(P, b, rowp, pres, rep, T, m_f, invZ, 1, (uint32_t)b0, L, ktok, tok, unused);
      f32_prefix(L, 1, sh);
      int b1 = f32_next(L, 1, -1, true, (uint32_t)b0, c0, m0, T, m_f, invZ, a.backend, tk, mp, thr_minp, tp, sh);
      for (int t1 = 0; t1 < 3 && b1 >= 0 && !found; ++t1) {
        const uint32_t prefix = ((uint32_t)b0 << 11) | (uint32_t)b1;
        f32_pass<ALIGNED>(P, b, rowp, pres, rep, T, m_f, invZ, 2, prefix, L, ktok, tok, unused);
        found = f32_walk(L, prefix, c0 + L.pcnt[1][b1], m0 + L.pmass[1][b1], T, m_f, invZ, a.backend, tk, mp,
                         thr_minp, tp, sh);
        if (!found)
          b1 = f32_next(L, 1, F32_BINS - 1 - b1, false, (uint32_t)b0, c0, m0, T, m_f, invZ, a.backend, tk, mp,
                        thr_minp, tp, sh);
      }
      if (!found)
        b0 = f32_next(L, 0, F32_BINS - 1 - b0, false, 0u, 0ull, 0ull, T, m_f, invZ, a.backend, tk, mp, thr_minp,
                      tp, sh);
    }
    return found;
  };
  float top_p_eff = top_p;
  if (a.backend == DSV_BACKEND_FLASHINFER && min_p > 0.f) {
    // flashinfer's min-p branch: top-p on the mass renormalised over the top-k (S_k from a
    // rank-only descent; no rank cut: the whole mass)
    const bool kf = descend(topk, 0.f, INFINITY);
    const double Sk = kf ? sh.cut_S : (double)(L.pmass[0][0] + L.mass[0][0]) / FX_ONE;
    top_p_eff = (float)((double)top_p * Sk);
    __syncthreads();  // (sh.cut_S read before the next descent)
  }
  const bool found = descend(topk, min_p, top_p_eff);
  // A cut that keeps only some of the cut key's values: each chunk's count of them, so that the
  // dense writer ranks a chunk's ties from the earlier chunks' counts
  const uint32_t cut_key = sh.cut_key;
  const int32_t cut_tie = sh.cut_tie;
  const bool count_ties = found && cut_tie > 0 && cut_tie != INT_MAX;
  if (count_ties) {
    constexpr int FE = Span<DSV_F32, NUC_THREADS>::FE;
    for (int c = 0; c < P.C; ++c) {
      const int64_t jlo = (int64_t)c * Elems<DSV_F32>::chunk + (int64_t)tid * FE;
      uint64_t t = 0;
      for_span<DSV_F32, ALIGNED, NUC_THREADS>(P, b, rowp, c, pres, rep, [&](int i, float x) {
        t += (jlo + i < V && key_of<DSV_F32>(x) == cut_key) ? 1u : 0u;
      });
      t = block_sum<NUC_WAVES>(t, sh.u);
      if (tid == 0) P.rties[r * NCHK + c] = (int32_t)t;
    }
  }
  if (tid < WAVE) {
    if (found) {
      rs.vcut = cut_key;
      rs.ktie = cut_tie;
      rs.S_kept = sh.cut_S;
    } else {  // every value is kept
      rs.vcut = 0u;
      rs.ktie = INT_MAX;
      rs.S_kept = (double)(L.pmass[0][0] + L.mass[0][0]) / FX_ONE;
    }
    rs.S_f = (float)rs.S_kept;
    if (count_ties) rs.flags |= FLAG_TIES_COUNTED;
    nucleus_finish<DSV_F32>(P, r, b, s, rs, T, xt, tok, tie_tok, ro);
  }
  __syncthreads();
}

// The i-th full-histogram row in row order goes to workgroup i % gridDim.x.
template <int DT, bool ALIGNED>
__global__ __launch_bounds__(NUC_THREADS) void k_nuc(KParams P) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ NucShared sh;
  const dsv_verify_args& a = P.a;
  uint32_t* hist = reinterpret_cast<uint32_t*>(dyn);
  // the rows the merge listed (a count, then row ids; their order does not affect any row)
  int n = P.nuc_rows[0];
  n = n < 0 ? 0 : (n > a.rows ? (int)a.rows : n);
  for (int i = blockIdx.x; i < n; i += gridDim.x) {
    const int32_t row = P.nuc_rows[1 + i];
    if (row < 0 || row >= a.rows) continue;
    if constexpr (DT == DSV_BF16) {
      nuc_row<DT, ALIGNED>(P, row, hist, sh, blockIdx.x, nullptr);
    } else {
      __shared__ F32NucShared fsh;
      nuc_row_f32<ALIGNED>(P, row, *reinterpret_cast<F32NucLds*>(dyn), fsh, nullptr);
    }
  }
}

// ---------------------------------------------------------------------------------------
// k_chunk: one pass over a 20480-value (bf16) / 12288-value (fp32) chunk held in registers
// ---------------------------------------------------------------------------------------
template <int DT, bool ALIGNED>
__global__ __launch_bounds__(CT, ALIGNED ? (DT == DSV_BF16 ? 7 : 6) : 5) void k_chunk(KParams P) {
  constexpr int n = Elems<DT>::n, CV = Elems<DT>::cv;
  constexpr int CHE = Elems<DT>::chunk;
  // nucleus rows: 32-bit value counts of the window; list rows: staged vectors, their ids, the
  // candidates and the radix counts (below); first the penalty step's slots (below)
  __shared__ uint4 big[HWIN / 4];
  __shared__ uint64_t su[CT / WAVE];
  __shared__ double sd[CT / WAVE];
  // history-hit vectors and masks of each wave: the penalty step is done, in every wave,
  // before the barriers of the chunk's max, which precede every other use of big
  uint4* const s_hv = big;
  uint32_t* const s_hm = reinterpret_cast<uint32_t*>(big + CT / WAVE * WHITV);
  static_assert(CT / WAVE * WHITV * 5 / 4 <= HWIN / 4, "penalty slots exceed the window buffer");
  __shared__ uint32_t s_pb[CHE / 32];  // the chunk's slice of the request's history bitmap
  __shared__ int32_t s_cnt, s_nq;
  __shared__ uint32_t s_wlo;
  __shared__ uint32_t s_kth;  // list rows: the key of the chunk's K-th largest value
  __shared__ float s_xtok;
  __shared__ int32_t s_arg;  // the chunk's first argmax id, from the thread that holds it
  const dsv_verify_args& a = P.a;
  const int C = P.C;
  const int64_t r = blockIdx.x / C;
  const int c = (int)(blockIdx.x - r * C);
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
  const int64_t V = a.vocab;
  const int64_t lo = (int64_t)c * CHE;
  const int64_t hi = lo + CHE < V ? lo + CHE : V;
  const char* rowp = row_ptr(a, r);
  const int64_t v0 = lo / n;
  // The request's history ids go out ahead of the chunk when the request is known without a
  // load (dense layout) and the history is short: the chunk's slice of the history bitmap is
  // then built while the chunk's loads are in flight.
  constexpr int HPRE = 4;  // history ids a thread loads ahead
  const bool hist_ahead =
      P.softmax && P.pbits && !P.force_greedy && !a.row_offsets && a.hist_len <= HPRE * CT;
  int32_t hid[HPRE];
  if (hist_ahead) {
    const int32_t* h = a.hist_ids + (int64_t)((uint32_t)r / (uint32_t)a.T) * a.hist_len;
#pragma unroll
    for (int k = 0; k < HPRE; ++k) hid[k] = k * CT + tid < a.hist_len ? h[k * CT + tid] : -1;
  }
  // the chunk's loads go out first, unconditionally (addresses clamped into the row); the
  // row's request and mode are looked up under them
  uint4 v[CV];
  const int64_t nfull = hi / n;  // vectors wholly inside the row end before this one
  if constexpr (ALIGNED) {
    // vectors past the row's end read as zeros here and are filled below
    const auto rs = buf_rsrc(rowp + lo * (16 / n), (uint32_t)((hi - lo) * (16 / n)));
#pragma unroll
    for (int u = 0; u < CV; ++u) v[u] = buf_load16(rs, (uint32_t)tid * 16u, (uint32_t)(u * CT * 16));
  } else {
#pragma unroll
    for (int u = 0; u < CV; ++u) v[u] = load_vec<DT>(rowp, v0 + (int64_t)u * CT + tid, hi, false);
  }
  if (hist_ahead) {
    for (int i = tid; i < CHE / 32; i += CT) s_pb[i] = 0u;
    __syncthreads();
    // (offsets into the chunk in 32-bit arithmetic: ids below lo wrap past the chunk's extent)
    const uint32_t ext = (uint32_t)(hi - lo);
#pragma unroll
    for (int k = 0; k < HPRE; ++k) {
      const uint32_t o = (uint32_t)hid[k] - (uint32_t)lo;
      if (o < ext) atomicOr(&s_pb[o >> 5], 1u << (o & 31));
    }
    __syncthreads();
  }
  int b = 0, s = 0;
  int mode = M_GREEDY;
  if (!P.force_greedy) {
    if (P.softmax) {
      if (!row_request(a, r, b, s)) return;
      b = __builtin_amdgcn_readfirstlane(b);
      s = __builtin_amdgcn_readfirstlane(s);
      mode = row_mode(a, b, 0);
    } else {
      mode = M_LIST;  // top-k rows
    }
  }
  // The row's parameters, loaded while the chunk's vector loads are in flight: the fence keeps
  // the compiler from sinking them into the mode sections, where each would be a dependent
  // load of its own behind the chunk's work.
  const bool pen = P.softmax && P.pbits != nullptr;
  float T = 1.f, top_p = 1.f, pres = 0.f, rep = 1.f;
  int topk = P.kcand;
  int64_t tok = -1;
  if (P.softmax && !P.force_greedy) {
    if (mode != M_GREEDY) T = a.temperatures[b];
    topk = a.top_ks[b];
    if (a.filter || a.sparse_joint) top_p = a.top_ps[b];
    if (pen) {
      pres = a.presence ? a.presence[b] : 0.f;
      rep = a.repetition ? a.repetition[b] : 1.f;
    }
    if (mode != M_GREEDY) tok = step_token(a, b, s);
  }
  asm volatile("" ::"s"(T), "s"(top_p), "s"(pres), "s"(rep), "s"(topk), "s"(tok));
  ChunkStat* st = P.cstat + r * C + c;
  if (ALIGNED && hi - lo < CHE) {
    // the row's last chunk: -inf past the row, and the partial last vector element by element
    const uint32_t fill = DT == DSV_BF16 ? FILL_BF16 : FILL_F32;
    const int64_t rel = nfull - v0;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      const int64_t vi = v0 + (int64_t)u * CT + tid;
      if (vi >= nfull) v[u] = make_uint4(fill, fill, fill, fill);
      if (hi % n && u == rel / CT && tid == rel % CT) v[u] = load_vec<DT>(rowp, nfull, hi, false);
    }
  }

  if (pen) {
    // History hits (about 0.3% of the values), penalised in place by penalize_hits.
    // The chunk's slice of the request's history bitmap, built from the history ids (here,
    // unless they went out ahead of the chunk: their loads queue behind the chunk's, which the
    // penalties wait for anyway); the workgroups of the request's first row store it for the
    // later kernels at the end.
    if (!hist_ahead) {
      for (int i = tid; i < CHE / 32; i += CT) s_pb[i] = 0u;
      __syncthreads();
      const int32_t* h = a.hist_ids + (int64_t)b * a.hist_len;
      const uint32_t ext = (uint32_t)(hi - lo);
      for (int i = tid; i < a.hist_len; i += CT) {
        const uint32_t o = (uint32_t)h[i] - (uint32_t)lo;
        if (o < ext) atomicOr(&s_pb[o >> 5], 1u << (o & 31));
      }
      __syncthreads();
    }
    // the n bits of vector u: bit (u CT + tid) n of the slice (lo is a multiple of 32)
    uint32_t bits[CV];
    {
      // vector u's word is u CT n / 32 words past vector 0's (CT n a multiple of 32)
      static_assert((CT * n) % 32 == 0, "vector rows of the bitmap slice are whole words");
      const uint32_t sh = (uint32_t)(tid * n) & 31u;
      const uint32_t* pbt = s_pb + ((tid * n) >> 5);
#pragma unroll
      for (int u = 0; u < CV; ++u) bits[u] = (pbt[u * (CT * n / 32)] >> sh) & ((1u << n) - 1u);
    }
    penalize_hits<DT, CV>(v, bits, pres, rep, s_hv + wid * WHITV, s_hm + wid * WHITV);
  }

  // the draft token's adjusted value, from the registers of the thread that holds it (read by
  // thread 0 and the nucleus pass after the softmax sum's barriers)
  const bool tok_here = tok >= lo && tok < hi;
  if (tok_here) {
    const int rel = (int)(tok - lo);
    const int vi = rel / n, uu = vi / CT;
    if (tid == vi - uu * CT) {
      uint4 w = v[0];
#pragma unroll
      for (int u = 1; u < CV; ++u)
        if (u == uu) w = v[u];
      s_xtok = vec_elem_dyn<DT>(w, rel - vi * n);
    }
  }

  // max and the first index attaining it
  float m_t = -INFINITY;
  int bu = -1;
  bool done = false;
  if constexpr (DT == DSV_BF16) {
    // bf16 bits compared as signed 16-bit integers (two a packed max): the order of the values
    // when the maximum is positive; a thread whose maximum is not takes the float path below
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    int best = INT_MIN;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      const s16x2 a = __builtin_elementwise_max(__builtin_bit_cast(s16x2, v[u].x), __builtin_bit_cast(s16x2, v[u].y));
      const s16x2 c = __builtin_elementwise_max(__builtin_bit_cast(s16x2, v[u].z), __builtin_bit_cast(s16x2, v[u].w));
      const s16x2 d = __builtin_elementwise_max(a, c);
      const int vm = (int)d.x > (int)d.y ? (int)d.x : (int)d.y;
      if (vm > best) {
        best = vm;
        bu = u;
      }
    }
    done = best > 0;
    if (done) m_t = __uint_as_float((uint32_t)best << 16);
  }
  if (!done) {
    bu = -1;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      float vm = vec_elem<DT>(v[u], 0);
#pragma unroll
      for (int e = 1; e < n; ++e) vm = fmaxf(vm, vec_elem<DT>(v[u], e));
      if (vm > m_t) {
        m_t = vm;
        bu = u;
      }
    }
  }
  // the chunk's max and the first vector holding it (the thread's first such vector, then the
  // lowest vector index over the workgroup: vectors are id-ordered); the element within it is
  // found by that vector's owner alone, which stores it with the statistics at the end
  const uint64_t cbest =
      block_max_u64<CT / WAVE>(bu >= 0 ? pack(key_of<DT>(m_t), v0 + (int64_t)bu * CT + tid) : 0ull, su);
  if (cbest && (uint32_t)(unpack_id(cbest) - v0) % CT == (uint32_t)tid) {
    uint4 w = v[0];
#pragma unroll
    for (int u = 1; u < CV; ++u)
      if (u == bu) w = v[u];
    int e0 = n - 1;
#pragma unroll
    for (int e = n - 1; e >= 0; --e)
      if (vec_elem<DT>(w, e) == m_t) e0 = e;
    s_arg = unpack_id(cbest) * n + e0;
  }
  reg_fence(v);
  ChunkStat out;
  out.m = cbest ? value_of_key<DT>(unpack_key(cbest)) : -INFINITY;
  out.arg = INT_MAX;  // (stored from s_arg by its owner, at the end)
  out.s = 0.0;
  out.ncand = 0;
  out.tieq = 0;
  out.wlo = WIN_EMPTY;
  out.kx = 0u;
  out.xtok = 0.f;
  out.pad = 0;

  // the softmax partial sum (support-list rows of the step only when their top-p test needs Z)
  if (P.softmax && mode != M_GREEDY && cbest && (mode != M_LIST || list_needs_z(a, top_p))) {
    const float c2 = log2e_over(T);
    const float mc2 = out.m * c2;
    float st_ = 0.f;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      reg_fence1(v[u], st_);
#pragma unroll
      for (int e = 0; e < n; ++e) st_ += __builtin_amdgcn_exp2f(fmaf(vec_elem<DT>(v[u], e), c2, -mc2));
    }
    out.s = block_sum<CT / WAVE>((double)st_, sd);
    reg_fence(v);
  }

  if (DT == DSV_BF16 && mode == M_HIST) {
    if constexpr (DT == DSV_BF16) {
      // counts of the values in the window [wlo, kmax] where the row's cut is expected: wlo is
      // the higher of kmax - (HWIN - 1) and the lowest key whose probability estimate
      // exp((x - m) / T) / (s + (C - 1)(s - 1)) reaches 2 (1 - top_p) / V -- the chunk's values
      // other than its maximum (whose term is 1) standing for each of the row's other chunks, so
      // that a chunk holding a dominant peak does not take the peak for every chunk's mass.  The
      // row merge takes the cut from the counts when it lies in every chunk's window, and the
      // full-histogram path otherwise.
      uint32_t* cnt = reinterpret_cast<uint32_t*>(big);
      if (wid == 0) {
        uint32_t wlo = WIN_EMPTY;
        if (cbest) {
          const uint32_t kmax = unpack_key(cbest);
          uint32_t kb = 0x80u;  // the lowest finite key
          const double z_est = out.s * (double)C - (double)(C - 1);
          const float floor_e = 2.f * (1.f - top_p) / (float)V * (float)(z_est > 1.0 ? z_est : 1.0);
          if (floor_e > 0.f && kmax > 0x80u) {
            const float c2 = log2e_over(T);
            // the closed form's key, x = m + log2(floor) / c2, as the search's guess
            const uint32_t guess = key_of<DT>(out.m + __builtin_amdgcn_logf(floor_e) / c2);
            kb = wave_first_key_near(0x80u, kmax, guess, [&](uint32_t k) {
              return __builtin_amdgcn_exp2f((value_of_key<DT>(k) - out.m) * c2) >= floor_e;
            });
          }
          const uint32_t wfloor = kmax >= (uint32_t)HWIN - 1u ? kmax - ((uint32_t)HWIN - 1u) : 0u;
          wlo = kb > wfloor ? kb : wfloor;
        }
        if (lane == 0) s_wlo = wlo;
      }
#pragma unroll
      for (int i = tid; i < HWIN / 4; i += CT) big[i] = make_uint4(0u, 0u, 0u, 0u);
      __syncthreads();
      const uint32_t wlo = s_wlo;
      int tq = 0;
      if (tok_here) {  // values equal to the draft token's ahead of it
        const float xtv = s_xtok;
        // element e of vector u is ahead of tok iff u * CT * n + e < rel
        const int64_t rel64 = tok - (v0 + tid) * n;
        const int rel = (int)(rel64 < 0 ? 0 : (rel64 > CV * CT * n ? CV * CT * n : rel64));
#pragma unroll
        for (int u = 0; u < CV; ++u) {
          order_after(v[u], tq);
#pragma unroll
          for (int e = 0; e < n; ++e) tq += (vec_elem<DT>(v[u], e) == xtv) & (u * CT * n + e < rel);
        }
      }
      uint32_t kx = 0u;
      if (wlo != WIN_EMPTY) {
        const uint32_t W = unpack_key(cbest) - wlo + 1u;
        if (wlo > 0x8000u) {
          // a window of positive values: position = raw bits - (wlo - 0x8000); zero, negative
          // and lower values fall outside.  The largest value below the window is not
          // tracked here (the merge takes the full-histogram path if it needs it).
          const uint32_t cb = wlo - 0x8000u;
          const uint32_t cb2 = cb | (cb << 16);
          // the increment and the byte-offset shift held in registers for the whole loop (the
          // compiler would otherwise materialise both for every element)
          uint32_t one = 1u, two = 2u;
#pragma unroll
          for (int u = 0; u < CV; ++u) {
            // (redefines the two constants after vector u is read, which orders this vector's
            // counts after the previous one's without redefining the vector itself: a copy of
            // every vector at the branch's join otherwise)
            asm volatile("" : "+v"(one), "+v"(two) : "v"(v[u].x), "v"(v[u].y), "v"(v[u].z), "v"(v[u].w));
            const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t o2 = sub_u16x2(w4[q], cb2);
              const uint32_t o0 = o2 & 0xffffu, o1 = o2 >> 16;
              if (o0 < W) __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(cnt) + (o0 << two)), one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
              if (o1 < W) __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(cnt) + (o1 << two)), one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
          }
          kx = KX_UNKNOWN;
        } else {
#pragma unroll
          for (int u = 0; u < CV; ++u) {
            reg_fence1(v[u]);
#pragma unroll
            for (int e = 0; e < n; ++e) {
              const uint32_t k = key_of<DT>(vec_elem<DT>(v[u], e));
              const uint32_t o = k - wlo;
              if (o < W)
                atomicAdd(&cnt[o], 1u);
              else
                kx = k > kx ? k : kx;
            }
          }
        }
      }
      kx = (uint32_t)block_max_u64<CT / WAVE>((uint64_t)kx, su);  // (its barriers order the counts)
      out.tieq = tok_here ? block_sum<CT / WAVE>(tq, reinterpret_cast<int*>(sd)) : 0;
      if (wlo != WIN_EMPTY) {
        // 16-bit counts (a chunk holds fewer than 65536 values), two keys a word
        const int nw = (int)((unpack_key(cbest) - wlo) >> 1) + 1;
        uint32_t* dst = P.hpart + (r * C + c) * (int64_t)(HWIN / 2);
        for (int i = tid; i < nw; i += CT) dst[i] = cnt[2 * i] | (cnt[2 * i + 1] << 16);
      }
      out.wlo = wlo;
      out.kx = kx;
    }
  } else if (mode == M_LIST) {
    // (sparse joint rows: the capacity + 1 largest, whatever the request's top-k <= capacity)
    int K = (P.softmax && a.sparse_joint) ? SJ_CAP + 1 : topk;
    K = K < 1 ? 1 : (K > P.kcand ? P.kcand : K);
    // admission bound: min over the 4 waves of each wave's ceil(K/4)-th largest thread-max key,
    // so that at least K values of the chunk are at or above it
    const int J = (K + (CT / WAVE) - 1) / (CT / WAVE);
    const uint32_t kt = key_of<DT>(m_t);
    const uint32_t wk = wave_kth_key<DT == DSV_BF16 ? 16 : 32>(kt, J);
    if (!P.softmax) __syncthreads();  // (softmax rows: the sum's barriers follow the last use of su)
    if (lane == 0) su[wid] = wk;
    if (tid == 0) {
      s_cnt = 0;
      s_nq = 0;
    }
    __syncthreads();
    uint32_t thr = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < CT / WAVE; ++i) thr = (uint32_t)su[i] < thr ? (uint32_t)su[i] : thr;
    // A positive bound (the usual case): a value reaches it iff its bits, as a signed integer
    // of the value's width, reach the bound's value bits (negative values are negative
    // integers); its key is then bits | the sign bit.
    constexpr uint32_t SIGNB = DT == DSV_BF16 ? 0x8000u : 0x80000000u;
    const bool pos_thr = thr > SIGNB;
    const int t0 = (int)(thr - SIGNB);
    auto sbits = [&](const uint4& w, int e) -> int {
      if constexpr (DT == DSV_BF16)
        return (int)(int16_t)bf16_bits(w, e);
      else
        return (int)(e == 0 ? w.x : e == 1 ? w.y : e == 2 ? w.z : w.w);
    };
    // the list pass's LDS, in big (the penalty slots there are done with)
    uint4* const stage = big;  // the vectors holding a value at or above the bound
    int16_t* const s_qid = reinterpret_cast<int16_t*>(big + STAGE_VECS);  // tid | vector << 8
    uint32_t* const hist256 = reinterpret_cast<uint32_t*>(big + STAGE_VECS + STAGE_VECS / 8);
    uint64_t* const cbuf = reinterpret_cast<uint64_t*>(big + STAGE_VECS + STAGE_VECS / 8 + 64);
    static_assert(STAGE_VECS + STAGE_VECS / 8 + 64 + CAND_CAP / 2 <= HWIN / 4, "list pass exceeds the window buffer");
    static_assert(CT <= 256 && CV <= 127, "stage ids are 16-bit");
    // only the threads whose max reaches the bound hold admitted values: they stage those of
    // their vectors that reach it (usually one) and the whole workgroup scans them
    uint32_t qm = 0u;  // the thread's vectors holding a value at or above the bound
    if (kt >= thr) {
#pragma unroll
      for (int u = 0; u < CV; ++u) {
        bool hit = false;
        if (pos_thr && DT == DSV_BF16) {
          typedef short s16x2 __attribute__((ext_vector_type(2)));
          const s16x2 a = __builtin_elementwise_max(__builtin_bit_cast(s16x2, v[u].x), __builtin_bit_cast(s16x2, v[u].y));
          const s16x2 c2 = __builtin_elementwise_max(__builtin_bit_cast(s16x2, v[u].z), __builtin_bit_cast(s16x2, v[u].w));
          const s16x2 d = __builtin_elementwise_max(a, c2);
          hit = ((int)d.x > (int)d.y ? (int)d.x : (int)d.y) >= t0;
        } else if (pos_thr) {
          hit = max(max((int)v[u].x, (int)v[u].y), max((int)v[u].z, (int)v[u].w)) >= t0;
        } else if constexpr (DT == DSV_F32) {
          // float bits as signed integers with the negative values' magnitude bits flipped
          // order as their keys do (key = image ^ 2^31), -0 one below +0; a zero bound (the key
          // of +-0) is lowered by one to take -0 in
          const int tb = (int)(thr ^ 0x80000000u);
          const int tl = tb == 0 ? -1 : tb;
          const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
          int s4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) s4[e] = (int)(w4[e] ^ ((uint32_t)((int)w4[e] >> 31) >> 1));
          const int mx = max(max(s4[0], s4[1]), max(s4[2], s4[3]));
          hit = mx >= tl;
        } else {
#pragma unroll
          for (int e = 0; e < n; ++e) hit |= key_of<DT>(vec_elem<DT>(v[u], e)) >= thr;
        }
        qm |= (uint32_t)hit << u;
      }
    }
    {
      const int nv = __popc(qm);
      const int incl = wave_incl_scan(nv);
      const int tot = readlane<WAVE - 1>(incl);
      int base = 0;
      if (lane == 0 && tot) base = atomicAdd(&s_nq, tot);
      int at = readlane<0>(base) + incl - nv;
#pragma unroll
      for (int u = 0; u < CV; ++u) {
        if ((qm >> u) & 1u) {
          if (at < STAGE_VECS) {
            stage[at] = v[u];
            s_qid[at] = (int16_t)(tid | (u << 8));
          }
          ++at;
        }
      }
    }
    __syncthreads();
    const int nq = s_nq;
    if (nq <= STAGE_VECS) {
      for (int vb = 0; vb < nq; vb += CT) {
        const int vi = vb + tid;
        uint4 w = make_uint4(0u, 0u, 0u, 0u);
        int64_t j0 = hi;
        if (vi < nq) {
          const int q = s_qid[vi];
          w = stage[vi];
          j0 = (v0 + (int64_t)(q >> 8) * CT + (q & 255)) * n;
        }
        uint32_t am = 0u;  // the vector's admitted elements
        if (pos_thr) {
#pragma unroll
          for (int e = 0; e < n; ++e) am |= (uint32_t)(sbits(w, e) >= t0) << e;
          const int64_t nval = hi - j0;  // elements of the vector inside the row
          am &= nval >= n ? (1u << n) - 1u : (nval <= 0 ? 0u : (1u << (uint32_t)nval) - 1u);
        } else {
#pragma unroll
          for (int e = 0; e < n; ++e)
            am |= (uint32_t)(key_of<DT>(vec_elem<DT>(w, e)) >= thr && j0 + e < hi) << e;
        }
        // slots: a prefix over the wave (DPP scan) and one LDS atomic a wave
        const int na = __popc(am);
        const int incl = wave_incl_scan(na);
        const int tot = readlane<WAVE - 1>(incl);
        if (tot) {
          int base = 0;
          if (lane == 0) base = atomicAdd(&s_cnt, tot);
          int at = readlane<0>(base) + incl - na;
#pragma unroll
          for (int e = 0; e < n; ++e) {
            if ((am >> e) & 1u) {
              const uint32_t key = pos_thr ? ((uint32_t)sbits(w, e) & (SIGNB | (SIGNB - 1u))) | SIGNB : key_of<DT>(vec_elem<DT>(w, e));
              if (at < CAND_CAP) cbuf[at] = pack(key, j0 + e);
              ++at;
            }
          }
        }
      }
    }
    __syncthreads();
    int nb = __builtin_amdgcn_readfirstlane(s_cnt);
    bool refilled = false;
    if (nq > STAGE_VECS || nb > CAND_CAP) {
      // too many vectors to stage, or too many admitted values: re-read the chunk
      nb = refill_candidates<DT>(pen ? s_pb : nullptr, rowp, lo, hi, K, pres, rep, cbuf,
                                 hist256, su, &s_cnt, nq > STAGE_VECS ? ((uint64_t)thr << 32) | 1ull : 0ull);
      refilled = true;
    }
    const int kk = K < nb ? K : nb;
    uint64_t* dst = P.cand + (r * C + c) * (int64_t)P.kcand;
    if (nb <= WAVE) {
      if (wid == 0) {
        // the K largest of the admitted values, unordered (the row merge ranks them): one a
        // lane, the K-th largest key by a radix select, then the lowest ids of its ties
        const uint64_t v_i = lane < nb ? cbuf[lane] : 0ull;
        bool take = lane < nb;
        if (nb > K) {
          const uint32_t key_i = lane < nb ? unpack_key(v_i) : 0u;
          const uint32_t kth = wave_kth_key<DT == DSV_BF16 ? 16 : 32>(key_i, K);
          const int need = K - __popcll(__ballot(lane < nb && key_i > kth));
          const uint64_t ties = __ballot(lane < nb && key_i == kth);
          int ahead = 0;  // ties with a lower id (a larger packed value)
          for (uint64_t m = ties; m; m &= m - 1ull) {
            const int j = __ffsll((long long)m) - 1;
            const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v_i >> 32), j) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v_i, j);
            ahead += o > v_i;
          }
          take = key_i > kth || (key_i == kth && lane < nb && ahead < need);
          if (lane == 0) s_kth = kth;
        }
        const uint64_t tb = __ballot(take);
        if (take)
          dst[__builtin_amdgcn_mbcnt_hi((uint32_t)(tb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)tb, 0u))] = v_i;
      }
    } else {  // more than a wave of values: each ranked against all (values are distinct)
      for (int i = tid; i < nb; i += CT) {
        const uint64_t v_i = cbuf[i];
        int rank = 0;
        for (int j = 0; j < nb; ++j) rank += cbuf[j] > v_i;
        if (rank < kk) dst[rank] = v_i;
        if (rank == kk - 1) s_kth = unpack_key(v_i);
      }
    }
    out.ncand = kk;
    if (P.softmax && a.sparse_joint && nb > K) {
      // Sparse joint rows keep every value tied with the row's k-th, so the row merge needs the
      // chunk's values at its list's smallest key that the list left out: all the values at that
      // key (every one reached the admission bound; a refilled buffer may miss some, then the
      // chunk is counted again from memory) less those in the list (the list holds every value
      // above that key).
      __syncthreads();
      const uint32_t kth = s_kth;
      int eq = 0, gt = 0;
      for (int i = tid; i < nb; i += CT) {
        const uint32_t key = unpack_key(cbuf[i]);
        eq += key == kth;
        gt += key > kth;
      }
      if (refilled) eq = count_key_chunk<DT>(pen ? s_pb : nullptr, rowp, lo, hi, kth, pres, rep);
      const int32_t eg = block_sum<CT / WAVE>(eq | (gt << 20), reinterpret_cast<int32_t*>(sd));
      out.tieq = (eg & 0xFFFFF) - (kk - (eg >> 20));
    }
  }
  // The statistics: thread 0 writes all but the argmax id and the draft token's value, which
  // their owners store from their own LDS writes (no barrier: the fields are disjoint).
  if (cbest && (uint32_t)(unpack_id(cbest) - v0) % CT == (uint32_t)tid) st->arg = s_arg;
  if (tok_here && tid == (int)((tok - lo) / n) % CT) st->xtok = s_xtok;
  if (tid == 0) {
    st->m = out.m;
    st->s = out.s;
    st->ncand = out.ncand;
    st->tieq = out.tieq;
    st->wlo = out.wlo;
    st->kx = out.kx;
    st->pad = 0;
    if (!cbest) st->arg = INT_MAX;
    if (!tok_here) st->xtok = 0.f;
    // The row merge's per-call state, written after the last load (a store ahead of the row's
    // parameter loads would turn those scalar loads into vector loads queued behind the
    // chunk's): its list of full-histogram rows, and the request's merged-row count and
    // deferred flag.  Every chunk-0 workgroup writes the same values (the merge runs after the
    // chunk pass); a request without rows here is left to k_final.
    if (c == 0) {
      if (P.nuc_rows) P.nuc_rows[0] = 0;
      if (P.req_cnt) {
        P.req_cnt[b] = 0u;
        P.deferred[b] = 1u;
      }
    }
  }
  if (pen && s == 0) {  // the request's history bitmap for the later kernels (its first row)
    uint32_t* dst = P.pbits + (int64_t)b * P.pwords + (lo >> 5);
    const int words = (int)((hi - lo + 31) >> 5);
    for (int i = tid; i < words; i += CT) dst[i] = s_pb[i];
  }
}

// Float32 nucleus rows: the row statistics here, the cut by the radix descent of k_nuc (wave 0).
template <int DT>
__device__ __forceinline__ void defer_nucleus(const KParams& P, int64_t r, float T, const RowPre& pre, RowOut* ro) {
  if (threadIdx.x >= WAVE) return;
  const int lane = threadIdx.x;
  const int C = P.C;
  float m_l = -INFINITY;
  int32_t arg_l = INT_MAX;
  double s_l = 0.0;
  if (lane < C) {
    m_l = pre.cs[lane].m;
    arg_l = pre.cs[lane].arg;
    s_l = pre.cs[lane].s;
  }
  const float M = wave_max_f32(m_l);
  const uint64_t at_max = __ballot(lane < C && m_l == M);
  int32_t arg = readlane_at(arg_l, at_max ? __ffsll((long long)at_max) - 1 : 0);
  if (arg == INT_MAX) arg = 0;
  const float c2 = log2e_over(T);
  const double Z = wave_sum(m_l > -INFINITY ? s_l * (double)__builtin_amdgcn_exp2f((m_l - M) * c2) : 0.0);
  RowSum rs;
  rs.mode = M_HIST;
  rs.argmax = arg;
  rs.kmax = key_of<DT>(M);
  rs.vcut = 0u;
  rs.ktie = INT_MAX;
  rs.nlist = 0;
  rs.flags = FLAG_FULL_HIST;
  rs.norm = 0;
  rs.m_f = M / T;
  rs.invZ = (float)(1.0 / Z);
  rs.Z = Z;
  rs.S_kept = 1.0;
  rs.S_f = 1.f;
  rs.p_draft = 0.f;
  if (lane == 0) {
    ro->rs = rs;
    ro->ok = 0;
    ro->nuc = 1;
  }
}

// ---------------------------------------------------------------------------------------
// Bonus draw (sampling/sparse/accept.py:249-307 and :179-204; runtime/worker.py:1048-1089)
//
// The bonus of a request is drawn from its row at the accepted length a: max(P - q_a, 0) when
// draft a+1 was rejected (P when that residual has no mass), P when every draft was accepted,
// by inverse CDF in id order.  Which draw a row would make is fixed before a is known, so the
// row merge draws every row's token (k_final picks row a's): support-list rows over their list,
// dense rows (unfiltered, nucleus) by locating the chunk from chunk masses -- softmax partial
// sums at the row scale, or the nucleus window counts above the cut -- less the residual's
// reduction at the q ids, then scanning that one chunk in id order.  Rows whose cut the full
// histogram settles (k_nuc) are drawn in k_final the same way.  The draw's P is computed with
// exp2 (within a few float ulps of the reference's p / S); the accept test uses the exact P.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void write_outputs(const dsv_verify_args& a, int b, int acc, int64_t bonus) {
  const int T = a.T;
  for (int i = threadIdx.x; i < T; i += blockDim.x) {
    int64_t val = 0;
    if (i < acc)
      val = a.candidates[(int64_t)b * T + i + 1];
    else if (i == acc)
      val = bonus;
    a.output[(int64_t)b * T + i] = val;
    if (a.kv_slots) {
      int32_t slot = -1;
      if (i <= acc && a.page_table) {
        const int64_t pos = (int64_t)a.prefix_lens[b] + i;
        if (pos >= 0 && pos < a.page_cols) slot = a.page_table[(int64_t)b * a.page_stride + pos];
      }
      a.kv_slots[(int64_t)b * T + i] = slot;
    }
  }
  if (threadIdx.x == 0) {
    a.accept[b] = acc;
    a.commit[b] = acc + 1;
    a.bonus[b] = bonus;
    a.new_seq[b] = a.prefix_lens[b] + acc + 1;
  }
}

// The gathers behind a request's outputs -- the draft token after position i and the KV slot of
// position i -- for the positions i = threadIdx.x - WAVE of waves 1 on, issued before the accepted
// length is known; write_outputs_at then only picks among them.
struct OutGather {
  int64_t tok = 0;
  int32_t slot = -1;
};
__device__ __forceinline__ OutGather gather_outputs(const dsv_verify_args& a, int b, int i, int32_t plen) {
  OutGather g;
  if (i < 0 || i >= a.T) return g;
  if (i + 1 < a.T) g.tok = a.candidates[(int64_t)b * a.T + i + 1];
  if (a.kv_slots && a.page_table) {
    const int64_t pos = (int64_t)plen + i;
    if (pos >= 0 && pos < a.page_cols) g.slot = a.page_table[(int64_t)b * a.page_stride + pos];
  }
  return g;
}
// write_outputs with the gathers of gather_outputs (positions past the first FCT - WAVE gather here)
__device__ __forceinline__ void write_outputs_at(const dsv_verify_args& a, int b, int acc, int64_t bonus,
                                                 const OutGather& g, int stride, int32_t plen) {
  const int T = a.T;
  const int i0 = (int)threadIdx.x - WAVE;
  for (int i = i0; i0 >= 0 && i < T; i += stride) {
    const OutGather o = i == i0 ? g : gather_outputs(a, b, i, plen);
    a.output[(int64_t)b * T + i] = i < acc ? o.tok : (i == acc ? bonus : 0);
    if (a.kv_slots) a.kv_slots[(int64_t)b * T + i] = i <= acc ? o.slot : -1;
  }
  if (threadIdx.x == 0) {
    a.accept[b] = acc;
    a.commit[b] = acc + 1;
    a.bonus[b] = bonus;
    a.new_seq[b] = plen + acc + 1;
  }
}

// ---------------------------------------------------------------------------------------
// k_merge: one workgroup per row (the rank selection uses all threads, the rest wave 0).  The
// row's decision and bonus token are stored device-coherently, then the row bumps its request's
// counter; the workgroup that completes the count (every row of the request merged) writes the
// request's outputs when the row merges drew its token.  Requests whose accepted row is dense
// (the draw planned) or decided by the full histogram stay deferred: k_final resolves them.
// ---------------------------------------------------------------------------------------
// The request's outputs from its rows' decisions, when the row merges drew the token: the
// accepted length a is the first row whose draft was rejected (the last row ends every prefix),
// and row a's merge drew the bonus token (support-list and greedy rows).  A dense row at a
// (its draw planned: a scan of one chunk) or a full-histogram row before it leaves the request
// to k_final.
__device__ __forceinline__ void final_rows(const KParams& P, int b, DrawShared& sh) {
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int64_t row0 = request_row0(a, b);
  const int cap = req_cap(a, b);
  if (tid < WAVE) {
    int acc = cap - 1;
    int64_t drawn = 0;
    for (int s0 = 0; s0 < cap; s0 += WAVE) {
      const int s = s0 + lane;
      const int32_t ok = s < cap - 1 ? ld_dev(P.step_ok + row0 + s) : 0;
      const int64_t rb = s < cap ? ld_dev(P.rbonus + row0 + s) : 0;
      const uint64_t end = __ballot(s < cap && ok == 0);
      if (end) {
        const int l = __ffsll((long long)end) - 1;
        acc = s0 + l;
        drawn = readlane_at(rb, l);
        break;
      }
    }
    if (tid == 0) {
      sh.acc = acc;
      sh.bonus = drawn;
    }
  }
  __syncthreads();
  const int acc = sh.acc;
  const int64_t bonus = sh.bonus;
  if (bonus <= BONUS_PLAN) {
    // a planned draw: k_final scans the chunk; the accepted length and the chunk go with the
    // deferred flag (2 + a, chunk + 1 in the top byte), so that k_final loads them at once
    const int cpl = (int)(BONUS_PLAN - 1 - bonus);
    if (tid == 0 && acc + 2 < DEFER_ACC) P.deferred[b] = ((uint32_t)(cpl + 1) << 24) | (uint32_t)(acc + 2);
    return;
  }
  if (bonus < 0) return;  // (BONUS_LATER: k_final)
  write_outputs(a, b, acc, bonus);
  if (tid == 0) P.deferred[b] = 0u;
}

template <int DT, bool ALIGNED>
__global__ __launch_bounds__(CT, 4) void k_merge(KParams P) {
  __shared__ union {  // a row merges as a support list or as a nucleus, never both
    MergeShared ms;
    NucMergeShared ns;
  } mu;
  MergeShared& ms = mu.ms;
  NucMergeShared& ns = mu.ns;
  __shared__ DrawShared ds;
  __shared__ RowPre pre;
  __shared__ RowOut ro;
  __shared__ uint32_t s_last;
  const dsv_verify_args& a = P.a;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  int b, s;
  if (!row_request(a, r, b, s)) {
    if (tid == 0) {
      P.rowsum[r].mode = M_SKIP;
      P.step_ok[r] = 0;
    }
    return;
  }
  const int mode = row_mode(a, b, 0);
  const float T = a.temperatures[b];
  const int cap = req_cap(a, b);
  const bool resid = s < cap - 1;  // the row tests draft s+1, and ends the prefix when it is rejected
  const bool tests = a.candidates != nullptr && resid;
  // one round of reads before the merge: the chunk statistics, the draft token and its coin
  // (wave 0), the q lanes (wave 1)
  if (tid < WAVE) {
    if (lane < P.C) pre.cs[lane] = P.cstat[r * P.C + lane];
    if (lane == 0) {
      // the draft token and its coin, loaded before the verify length settles whether the row
      // tests one (positions clamped into the request's rows)
      int64_t tk = -1;
      float u = 0.f;
      if (a.candidates && a.T >= 2) {
        tk = a.candidates[(int64_t)b * a.T + (s + 1 < a.T ? s + 1 : a.T - 1)];
        u = a.uniforms[(int64_t)b * (a.T - 1) + (s < a.T - 1 ? s : a.T - 2)];
      }
      pre.tok = tests ? tk : -1;
      pre.u = tests ? u : 0.f;
      pre.uf = a.candidates ? a.uniform_final[b] : 0.f;
      pre.top_p = a.top_ps ? a.top_ps[b] : 1.f;
      pre.min_p = a.min_ps ? a.min_ps[b] : 0.f;
      pre.top_k = a.top_ks[b];
      pre.pres = P.pbits && a.presence ? a.presence[b] : 0.f;
      pre.rep = P.pbits && a.repetition ? a.repetition[b] : 1.f;
    }
  }
  // wave 1: the q lanes, and for dense rows the loads of the logits at their ids, which stay in
  // flight through the merge (the bonus plan is their first use)
  QxLoad ql;
  if (tid >= WAVE && tid < 2 * WAVE)
    fetch_q_wave<DT>(P, b, s, tests, row_ptr(a, r), mode == M_UNF || mode == M_HIST, ds, ql);
  __syncthreads();
  if (mode == M_HIST) {
    if constexpr (DT == DSV_BF16)
      merge_nucleus<DT>(P, r, b, s, T, ns, ds, pre, &ro);
    else
      defer_nucleus<DT>(P, r, T, pre, &ro);
  } else {
    merge_row<DT>(P, r, b, s, mode, T, ms, ds, pre, &ro);
  }
  if (tid >= WAVE && tid < 2 * WAVE) qx_finish<DT>(ql, pre.pres, pre.rep, ds);
  __syncthreads();
  // The bonus token this row gives when it is the request's accepted length: none for a row
  // whose draft was accepted before the last row (the accepted length lies beyond it), nor for
  // the target-distribution entry.
  const RowSum& rs = ro.rs;  // (read from LDS where used: fewer live registers)
  int64_t bonus = 0;
  if (!a.candidates || (resid && ro.ok)) {
  } else if (rs.mode == M_GREEDY) {
    bonus = rs.argmax;
  } else if (rs.mode == M_LIST) {
    bonus = tid < WAVE ? list_draw(a, resid, pre.uf, ds) : 0;
  } else if (rs.flags & (FLAG_FULL_HIST | FLAG_SCAN_DRAW)) {
    bonus = BONUS_LATER;
  } else {
    // dense rows: the chunk and threshold; k_final scans the chunk when this row is the accepted
    // one.  The plan, stored by waves 1 and 2: a wave's later waits cover only its own stores,
    // so the row's stores (wave 0, below) do not queue behind these.
    dense_plan<DT, ALIGNED, CT>(P, b, row_ptr(a, r), rs, T, pre.pres, pre.rep, resid, pre.uf, ds, true);
    static_assert(QMAX <= WAVE && CT >= 3 * WAVE, "plan stores by waves 1 and 2");
    DrawPlan* pl = P.plans + r;
    const int lq = (int)threadIdx.x - WAVE;
    if (lq >= 0 && lq < QMAX) pl->qd[lq] = ds.qd[lq];
    if (threadIdx.x == 2 * WAVE) {
      pl->thr = ds.thr;
      pl->chunk_lo = ds.chunk_lo;
      pl->chunk = ds.chunk;
      pl->tieq = ds.tieq;
      pl->use_r = ds.use_r;
      pl->pad = 0;
    }
    bonus = BONUS_PLAN - 1 - ds.chunk;  // (the chunk, for k_final's early loads)
  }
  if (tid == 0) {
    P.rowsum[r] = rs;
    st_dev(P.step_ok + r, ro.ok);
    if (a.candidates) st_dev(P.rbonus + r, bonus);
    if (ro.nuc) {
      const int32_t at = atomicAdd(&P.nuc_rows[0], 1);
      if (at < a.rows) P.nuc_rows[1 + at] = (int32_t)r;
    }
  }
  if (!a.candidates) return;  // (the target-distribution entries write no outputs)
  // the row's decision and token have reached the coherence point before the row is counted;
  // the workgroup that completes the request's count writes the request's outputs
  if (tid == 0) {
    publish_wait();
    s_last = atomicAdd(P.req_cnt + b, 1u) == (uint32_t)(cap - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (s_last) final_rows(P, b, ds);
}

// ---------------------------------------------------------------------------------------
// k_final: outputs, one workgroup per request the row merge left (only_deferred; else every
// request) -- the accepted length a, and the bonus token of row a (drawn by the row merge, or
// here for rows the full histogram settled)
// ---------------------------------------------------------------------------------------
template <int DT, bool ALIGNED>
__global__ __launch_bounds__(FCT) void k_final(KParams P) {
  constexpr int CHE = Elems<DT>::chunk;
  static_assert(FCT == NUC_THREADS, "k_final resolves full-histogram rows with the nucleus code");
  extern __shared__ __align__(16) unsigned char dyn[];  // (final_nuc: the full-histogram LDS)
  __shared__ DrawShared sh;
  __shared__ RowOut fro;  // a full-histogram row resolved here
  __shared__ uint4 s_hv[FCT / WAVE * WHITV];  // history-hit slots of the draw
  __shared__ uint32_t s_hm[FCT / WAVE * WHITV];
  const dsv_verify_args& a = P.a;
  // KF_ROLES workgroups a request: role 0 decides it; the others are helpers (below).  A
  // request's workgroups are bs apart, so for bs a multiple of 8 they share an XCD (and its L2).
  const int b = (int)(blockIdx.x % (unsigned)a.bs);
  const int role = (int)(blockIdx.x / (unsigned)a.bs);
  const uint32_t dfl = P.only_deferred ? P.deferred[b] : 1u;
  if (role != 0) {
    // A helper: when the row merge planned the request's draw (the accepted row and its chunk
    // ride in the deferred flag), a share of that chunk is read with the default cache policy,
    // so that the lines are in the caches when role 0 streams the chunk: one workgroup's reads
    // of 40 KB take several rounds of its own outstanding misses.
    if constexpr (ALIGNED) {
      if (dfl >= 2u) {
        constexpr int n = Elems<DT>::n, CHE = Elems<DT>::chunk;
        const int acc = (int)(dfl & (DEFER_ACC - 1)) - 2;
        const int cpl = (int)(dfl >> 24) - 1;
        const int64_t r = request_row0(a, b) + acc;
        if (cpl >= 0 && cpl < P.C && acc >= 0 && r >= 0 && r < a.rows) {
          const int64_t lo = (int64_t)cpl * CHE, hi = lo + CHE < a.vocab ? lo + CHE : a.vocab;
          const uint32_t bytes = (uint32_t)((hi - lo) * (16 / n));
          const auto rsr = buf_rsrc(row_ptr(a, r) + lo * (16 / n), bytes);
          const uint32_t nvec = (bytes + 15u) / 16u;
          const uint32_t part = (nvec + (KF_ROLES - 2)) / (KF_ROLES - 1);
          const uint32_t v0 = (uint32_t)(role - 1) * part, v1 = v0 + part < nvec ? v0 + part : nvec;
          uint32_t x = 0u;
          for (uint32_t v = v0 + threadIdx.x; v < v1; v += FCT) {
            const uint4 t = buf_load16_cached(rsr, v * 16u, 0u);
            x ^= t.x ^ t.y ^ t.z ^ t.w;
          }
          asm volatile("" ::"v"(x));
        }
      }
    }
    return;
  }
  if (dfl == 0u) {
    // the row merge wrote the request's outputs -- if the request has rows (its deferred flag
    // is set by the chunk pass of its own rows; one without is decided here)
    int b0 = -1, s0 = -1;
    const int64_t r0 = request_row0(a, b);
    if (r0 >= 0 && r0 < a.rows && row_request(a, r0, b0, s0) && b0 == b && s0 == 0) return;
  }
  const int tid = threadIdx.x, lane = tid & (WAVE - 1);
  const int64_t V = a.vocab;
  int64_t row0 = request_row0(a, b);
  int cap = req_cap(a, b);
  const bool rows_ok = row0 >= 0 && row0 < a.rows;
  if (!rows_ok) {  // inconsistent row offsets: no row of this request can be read
    write_outputs(a, b, 0, V - 1);
    return;
  }
  if (row0 + cap > a.rows) cap = (int)(a.rows - row0);
  const int32_t plen = a.prefix_lens[b];
  const OutGather og = gather_outputs(a, b, tid - WAVE, plen);
  // the request's parameters for a dense draw, read with the step decisions
  const float T = a.temperatures[b];
  const bool pen = P.pbits != nullptr;
  const float pres = pen && a.presence ? a.presence[b] : 0.f;
  const float rep = pen && a.repetition ? a.repetition[b] : 1.f;
  const float uf = a.uniform_final[b];
  // the first step from s_from on that ends the prefix (a rejected draft; the last row ends every
  // prefix) and the bonus its row's merge drew or planned, read together by wave 0
  auto scan = [&](int s_from) {
    if (tid < WAVE) {
      int acc = cap - 1;
      int64_t drawn = 0;
      for (int s0 = s_from; s0 < cap; s0 += WAVE) {
        const int s = s0 + lane;
        const int32_t ok = s < cap - 1 ? P.step_ok[row0 + s] : 0;
        const int64_t rb = s < cap ? P.rbonus[row0 + s] : 0;
        const uint64_t end = __ballot(s < cap && ok == 0);
        if (end) {
          const int l = __ffsll((long long)end) - 1;
          acc = s0 + l;
          drawn = readlane_at(rb, l);
          break;
        }
      }
      if (tid == 0) {
        sh.acc = acc;
        sh.bonus = drawn;
      }
    }
    __syncthreads();
  };
  int acc;
  int64_t bonus;
  if (dfl >= 2u) {  // the row merge's scan: a planned draw at a known accepted length
    acc = (int)(dfl & (DEFER_ACC - 1)) - 2;
    bonus = BONUS_PLAN - 1 - ((int64_t)(dfl >> 24) - 1);
  } else {
    scan(0);
    acc = sh.acc;
    bonus = sh.bonus;
  }
  bool own = false;  // the accepted row's RowSum is fro.rs (resolved here)
  if (P.final_nuc) {
    // A row whose cut the merge's windows did not settle carries a placeholder decision (0):
    // its full histogram decides it here, and the scan resumes after it when it accepts.
    while (bonus == BONUS_LATER) {
      const int64_t r = row0 + acc;
      if constexpr (DT == DSV_BF16) {
        __shared__ NucShared nsh;
        nuc_row<DT, ALIGNED>(P, r, reinterpret_cast<uint32_t*>(dyn), nsh, b, &fro);
      } else {
        __shared__ F32NucShared fsh;
        nuc_row_f32<ALIGNED>(P, r, *reinterpret_cast<F32NucLds*>(dyn), fsh, &fro);
      }
      __syncthreads();
      if (acc < cap - 1 && fro.ok) {
        scan(acc + 1);
        acc = sh.acc;
        bonus = sh.bonus;
        continue;
      }
      own = true;
      break;
    }
  }
  if (bonus <= BONUS_PLAN) {  // the row merge planned the draw: scan the chunk
    const int64_t rstar = row0 + acc;
    const bool resid = acc < cap - 1;
    const DrawPlan* pl = P.plans + rstar;
    // the planned chunk's loads go out first, beside the plan's
    const int cpl = (int)(BONUS_PLAN - 1 - bonus);  // (-1: no mass anywhere, no scan)
    Span<DT, FCT> sp;
    if (cpl >= 0) span_load<DT, ALIGNED, FCT>(P, b, row_ptr(a, rstar), cpl, sp);
    if (tid < WAVE) {
      // the plan and the q lanes of the rejected draft in one round (dense_pick's first barrier
      // publishes them): ids, clamped values, whether the lane is the last with its id
      const int64_t qi = ((int64_t)b * (a.T - 1) + acc) * a.K;
      const bool on = resid && lane < a.K;
      const int64_t qid = on ? load_index(a.q_ids, a.q_ids_i64, qi + lane) : -1;
      const float qv = on ? clamp01(a.q_values[qi + lane]) : 0.f;
      const double qd = pl->qd[lane];
      const int32_t ch = pl->chunk;
      if (lane == 0) {
        sh.thr = pl->thr;
        sh.chunk_lo = pl->chunk_lo;
        sh.chunk = ch;
        sh.tieq = pl->tieq;
        sh.use_r = pl->use_r;
      }
      sh.qid[lane] = qid;
      sh.qv[lane] = qv;
      sh.qd[lane] = qd;
      const bool last = q_last_lane(qid, a.K, V);
      sh.qlast[lane] = last;
      const uint64_t qm = __ballot(last && ch >= 0 && qid / CHE == ch);
      if (lane == 0) sh.qmask = qm;
    }
    const RowSum rs = P.rowsum[rstar];
    bonus = dense_pick<DT, ALIGNED, FCT, true>(P, b, row_ptr(a, rstar), rs, T, pres, rep, sh, sp, s_hv, s_hm);
  } else if (bonus == BONUS_LATER) {
    const int64_t rstar = row0 + acc;
    const RowSum rs = own ? fro.rs : P.rowsum[rstar];
    const bool resid = acc < cap - 1;
    stage_q(a, b, acc, resid, sh);
    const char* rowp = row_ptr(a, rstar);
    const BonusP bp = bonus_p<DT>(rs, T);
    for (int c = 0; c < P.C; ++c) {  // chunk masses: a scan of every chunk
      double m = 0.0;
      int32_t t = 0;
      for_span<DT, ALIGNED, FCT>(P, b, rowp, c, pres, rep, [&](int, float x) {
        const uint32_t k = key_of<DT>(x);
        if (rs.mode != M_HIST || k > rs.vcut)
          m += (double)bp(x);
        else if (k == rs.vcut)
          ++t;
      });
      m = block_sum<FCT / WAVE>(m, sh.red_d);
      t = block_sum<FCT / WAVE>(t, sh.red_i);
      if (tid == 0) {
        sh.cm[c] = m;
        sh.ct[c] = t;
      }
    }
    __syncthreads();
    dense_plan<DT, ALIGNED, FCT>(P, b, rowp, rs, T, pres, rep, resid, uf, sh);
    Span<DT, FCT> unused;
    bonus = dense_pick<DT, ALIGNED, FCT>(P, b, rowp, rs, T, pres, rep, sh, unused, s_hv, s_hm);
  }
  write_outputs_at(a, b, acc, bonus, og, FCT - WAVE, plen);
}

// ---------------------------------------------------------------------------------------
// The target distribution of one (row, chunk) written out densely with each thread a span of
// consecutive ids (runtime/worker.py:440-508): the ordered path of k_dense_p -- rows whose cut
// keeps only some of the values at the cut key (their rank in id order decides), and outputs
// that are not 16-byte aligned.
// ---------------------------------------------------------------------------------------
template <int DT, bool ALIGNED>
__device__ __forceinline__ void dense_p_spans(const KParams& P, int64_t r, int c, int b, const RowSum& rs, int mode,
                                              float* out, int64_t out_stride) {
  constexpr int CV = Elems<DT>::cv, CHE = Elems<DT>::chunk, FE = CV * Elems<DT>::n;
  constexpr int NW = CT / WAVE;
  __shared__ int32_t red_i[NW];
  __shared__ ListEntry lst[DSV_LIST_K];
  __shared__ int32_t s_before;
  const dsv_verify_args& a = P.a;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const int64_t jlo = (int64_t)c * CHE + (int64_t)tid * FE;
  float* orow = out + r * out_stride;
  // the span's values, four at a time
  float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
  auto put = [&](int i, float v) {
    const int k = i & 3;
    if (k == 0) acc4.x = v; else if (k == 1) acc4.y = v; else if (k == 2) acc4.z = v; else acc4.w = v;
    if (k == 3) {
      const int64_t j = jlo + i - 3;
      if (j + 3 < V) {
        *reinterpret_cast<float4*>(orow + j) = acc4;
      } else {
        if (j < V) orow[j] = acc4.x;
        if (j + 1 < V) orow[j + 1] = acc4.y;
        if (j + 2 < V) orow[j + 2] = acc4.z;
      }
    }
  };
  const bool vec_ok = (out_stride % 4 == 0) && ((uintptr_t)out % 16 == 0);
  auto put1 = [&](int i, float v) {  // unaligned output: element stores
    const int64_t j = jlo + i;
    if (j < V) orow[j] = v;
  };
  if (mode == M_SKIP || mode == M_GREEDY || mode == M_LIST) {
    int n = 0;
    if (mode == M_LIST) {
      n = rs.nlist;
      for (int i = tid; i < n; i += CT) lst[i] = P.lists[r * DSV_LIST_K + i];
      __syncthreads();
    }
    for (int i = 0; i < FE; ++i) {
      const int64_t j = jlo + i;
      float v = 0.f;
      if (mode == M_GREEDY)
        v = j == (int64_t)rs.argmax ? 1.f : 0.f;
      else if (mode == M_LIST)
        for (int e = 0; e < n; ++e)
          if ((int64_t)lst[e].id == j) {
            v = lst[e].P;
            if (P.raw_p && P.src_p) {  // the input probability itself
              v = P.src_p[r * P.src_stride + j];
            } else if (P.raw_p) {  // the unrenormalised p: recomputed from the adjusted logit
              float x = load_elem<DT>(row_ptr(a, r), j);
              if (P.pbits && pen_test(P, b, j))
                x = penalize<DT>(x, a.presence ? a.presence[b] : 0.f, a.repetition ? a.repetition[b] : 1.f);
              v = prob_of(x, a.temperatures[b], rs.m_f, rs.invZ);
            }
          }
      if (vec_ok) put(i, v); else put1(i, v);
    }
    return;
  }
  const bool pen = P.pbits != nullptr;
  const float pres = pen && a.presence ? a.presence[b] : 0.f;
  const float rep = pen && a.repetition ? a.repetition[b] : 1.f;
  const float T = a.temperatures[b];
  const char* rowp = row_ptr(a, r);
  const bool hist = mode == M_HIST;
  int32_t tbefore = 0;
  // the chunks' counts of the cut key's values are in rties (merged rows, and full-histogram rows
  // whose resolver counted them)
  const bool ties_known = !(rs.flags & FLAG_FULL_HIST) || (rs.flags & FLAG_TIES_COUNTED);
  if (hist && rs.ktie > 0 && rs.ktie != INT_MAX) {
    // the cut key's values before this thread's span, in id order
    int32_t t = 0;
    for_span<DT, ALIGNED, CT>(P, b, rowp, c, pres, rep, [&](int, float x) { t += key_of<DT>(x) == rs.vcut; });
    int32_t tot = 0;
    tbefore = block_excl_scan<NW>(t, red_i, &tot);
    if (tid == 0) {
      int32_t before = 0;
      if (ties_known) {
        for (int c2 = 0; c2 < c; ++c2) before += P.rties[r * NCHK + c2];
      } else {
        s_before = 0;
      }
      if (ties_known) s_before = before;
    }
    if (!ties_known) {  // (rare) the earlier chunks' counts by scanning them
      int32_t e = 0;
      for (int c2 = 0; c2 < c; ++c2)
        for_span<DT, ALIGNED, CT>(P, b, rowp, c2, pres, rep, [&](int, float x) { e += key_of<DT>(x) == rs.vcut; });
      e = block_sum<NW>(e, red_i);
      if (tid == 0) s_before = e;
    }
    __syncthreads();
    tbefore += s_before;
  }
  int32_t seen = 0;
  for_span<DT, ALIGNED, CT>(P, b, rowp, c, pres, rep, [&](int i, float x) {
    float v = 0.f;
    const uint32_t k = key_of<DT>(x);
    const bool kept = !hist || k > rs.vcut || (k == rs.vcut && (int64_t)tbefore + seen < (int64_t)rs.ktie);
    if (kept)
      v = P.raw_p ? (P.src_p ? (jlo + i < V ? P.src_p[r * P.src_stride + jlo + i] : 0.f)  // (ids past the row: -inf)
                             : prob_of(x, T, rs.m_f, rs.invZ))
                  : (float)dense_P(rs, T, x);
    seen += hist && k == rs.vcut;
    if (vec_ok) put(i, v); else put1(i, v);
  });
}


// ---------------------------------------------------------------------------------------
// k_dense_p: the target distribution written out densely (runtime/worker.py:440-508), one
// workgroup per (row, chunk).  The chunk's values are laid out as the chunk pass loads them
// (thread t, vector u: ids (u CT + t) n .. + n), so that a wave's loads and 16-byte stores are
// contiguous; support-list rows write zeros with the list's values at their ids (an LDS bitmap
// of the chunk's list ids), greedy rows the one-hot row.  Rows whose cut keeps only some of the
// values at the cut key (when the chunks' counts of them are unknown), and unaligned outputs,
// take the ordered path above.
// ---------------------------------------------------------------------------------------
template <int DT, bool ALIGNED>
__global__ __launch_bounds__(CT) void k_dense_p(KParams P, float* out, int64_t out_stride) {
  constexpr int n = Elems<DT>::n, CV = Elems<DT>::cv, CHE = Elems<DT>::chunk;
  constexpr int NW = CT / WAVE;
  __shared__ ListEntry lst[DSV_LIST_K];
  __shared__ uint32_t s_bm[CHE / 32];  // list rows: the chunk's list ids; softmax rows: history bits
  __shared__ uint4 s_hv[NW * WHITV];    // history-hit vectors of each wave
  __shared__ uint32_t s_hm[NW * WHITV];
  __shared__ int32_t s_wt[CV * NW];     // partial ties: each wave's cut-key values of vector u
  __shared__ int32_t s_before;          // partial ties: the cut-key values of the earlier chunks
  const dsv_verify_args& a = P.a;
  const int C = P.C;
  const int64_t r = blockIdx.x / C;
  const int c = (int)(blockIdx.x - r * C);
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
  const int64_t V = a.vocab;
  float* orow = out + r * out_stride;
  int b = 0, s = 0;
  const bool live_row = row_request(a, r, b, s);
  const RowSum rs = P.rowsum[r];
  const int mode = live_row ? rs.mode : M_SKIP;
  const bool hist = mode == M_HIST;
  const bool vec_ok = (out_stride % 4 == 0) && ((uintptr_t)out % 16 == 0);
  // a cut that keeps only the first ktie values of the cut key in id order (partial ties)
  const bool part_ties = hist && rs.ktie > 0 && rs.ktie != INT_MAX;
  if (!vec_ok || (part_ties && (rs.flags & FLAG_FULL_HIST) && !(rs.flags & FLAG_TIES_COUNTED))) {
    dense_p_spans<DT, ALIGNED>(P, r, c, b, rs, mode, out, out_stride);
    return;
  }
  const int64_t lo = (int64_t)c * CHE, hi = lo + CHE < V ? lo + CHE : V;
  const int64_t v0 = lo / n;
  // vector u's n values at ids j0 = (v0 + u CT + tid) n: 16-byte stores, element stores at the
  // row's end
  auto store_vec = [&](int64_t j0, const float (&x)[n]) {
    if (j0 + n <= hi) {
#pragma unroll
      for (int q = 0; q < n / 4; ++q)
        *reinterpret_cast<float4*>(orow + j0 + 4 * q) = make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
    } else {
#pragma unroll
      for (int e = 0; e < n; ++e)
        if (j0 + e < hi) orow[j0 + e] = x[e];
    }
  };
  if (mode != M_UNF && !hist) {  // skipped, greedy and support-list rows
    const int nl = mode == M_LIST ? rs.nlist : 0;
    if (mode == M_LIST) {
      for (int i = tid; i < CHE / 32; i += CT) s_bm[i] = 0u;
      for (int i = tid; i < nl; i += CT) lst[i] = P.lists[r * DSV_LIST_K + i];
      __syncthreads();
      for (int i = tid; i < nl; i += CT) {
        const uint32_t o = (uint32_t)lst[i].id - (uint32_t)lo;
        if (o < (uint32_t)(hi - lo)) atomicOr(&s_bm[o >> 5], 1u << (o & 31));
      }
      __syncthreads();
    }
    // No logits are read here, so the values go out as 4-float groups with a wave's lanes on
    // consecutive groups (16-byte stores a wave covers 1 KB with, where the 8-value vectors of
    // the softmax rows take two half-filled stores).  Chunk offsets in 32 bits; a group's
    // nonzero elements from one subtraction (greedy: the one-hot's offset, -1 for none) or one
    // bitmap nibble (support lists), the values only then
    constexpr int G = 4;
    const uint32_t ext = (uint32_t)(hi - lo);
    const uint32_t oh = mode == M_GREEDY ? (uint32_t)rs.argmax - (uint32_t)lo : 0xFFFFFFFFu;
#pragma unroll
    for (int u = 0; u < CHE / G / CT; ++u) {
      const uint32_t o0 = (uint32_t)((u * CT + tid) * G);
      if (o0 >= ext) continue;
      const int64_t j0 = lo + o0;
      float x[G];
#pragma unroll
      for (int e = 0; e < G; ++e) x[e] = 0.f;
      if (mode == M_GREEDY) {
        const uint32_t e1 = oh - o0;
        if (e1 < (uint32_t)G) {
#pragma unroll
          for (int e = 0; e < G; ++e) x[e] = (uint32_t)e == e1 ? 1.f : 0.f;
        }
      } else if (mode == M_LIST) {
        const uint32_t bits = (s_bm[o0 >> 5] >> (o0 & 31)) & ((1u << G) - 1u);
        if (bits) {
#pragma unroll
          for (int e = 0; e < G; ++e) {
            if (!((bits >> e) & 1u)) continue;
            const int64_t j = j0 + e;
            for (int q = 0; q < nl; ++q)
              if ((int64_t)lst[q].id == j) {
                x[e] = lst[q].P;
                if (P.raw_p && P.src_p) {  // the input probability itself
                  x[e] = P.src_p[r * P.src_stride + j];
                } else if (P.raw_p) {  // the unrenormalised p: recomputed from the adjusted logit
                  float xv = load_elem<DT>(row_ptr(a, r), j);
                  if (P.pbits && pen_test(P, b, j))
                    xv = penalize<DT>(xv, a.presence ? a.presence[b] : 0.f, a.repetition ? a.repetition[b] : 1.f);
                  x[e] = prob_of(xv, a.temperatures[b], rs.m_f, rs.invZ);
                }
              }
          }
        }
      }
      if (j0 + G <= hi) {
        *reinterpret_cast<float4*>(orow + j0) = make_float4(x[0], x[1], x[2], x[3]);
      } else {
#pragma unroll
        for (int e = 0; e < G; ++e)
          if (j0 + e < hi) orow[j0 + e] = x[e];
      }
    }
    return;
  }
  // softmax rows: the chunk in registers, as the chunk pass loads it
  const bool pen = P.pbits != nullptr;
  const float pres = pen && a.presence ? a.presence[b] : 0.f;
  const float rep = pen && a.repetition ? a.repetition[b] : 1.f;
  const float T = a.temperatures[b];
  const char* rowp = row_ptr(a, r);
  uint4 v[CV];
  const int64_t nfull = hi / n;
  if constexpr (ALIGNED) {
    const auto rsr = buf_rsrc(rowp + lo * (16 / n), (uint32_t)((hi - lo) * (16 / n)));
#pragma unroll
    for (int u = 0; u < CV; ++u) v[u] = buf_load16(rsr, (uint32_t)tid * 16u, (uint32_t)(u * CT * 16));
    if (hi - lo < CHE) {  // the row's last chunk: the partial last vector element by element
      const int64_t rel = nfull - v0;
#pragma unroll
      for (int u = 0; u < CV; ++u)
        if (hi % n && u == rel / CT && tid == rel % CT) v[u] = load_vec<DT>(rowp, nfull, hi, false);
    }
  } else {
#pragma unroll
    for (int u = 0; u < CV; ++u) v[u] = load_vec<DT>(rowp, v0 + (int64_t)u * CT + tid, hi, false);
  }
  if (pen) {
    for (int i = tid; i < CHE / 32; i += CT) {
      const int64_t w = (lo >> 5) + i;
      s_bm[i] = w < P.pwords ? pen_word(P, b, w) : 0u;
    }
    __syncthreads();
    static_assert((CT * n) % 32 == 0, "vector rows of the bitmap slice are whole words");
    uint32_t bits[CV];
    const uint32_t sh = (uint32_t)(tid * n) & 31u;
    const uint32_t* pbt = s_bm + ((tid * n) >> 5);
#pragma unroll
    for (int u = 0; u < CV; ++u) bits[u] = (pbt[u * (CT * n / 32)] >> sh) & ((1u << n) - 1u);
    penalize_hits<DT, CV>(v, bits, pres, rep, s_hv + wid * WHITV, s_hm + wid * WHITV);
  }
  // Partial ties: a cut-key value's rank in id order is the earlier chunks' count (the row
  // merge's per-chunk counts), the values of the vectors before its vector (vector index order
  // u CT + t is id order: a prefix over vectors u-major, from one wave scan a vector and the
  // waves' totals), then the ones before it in its vector.
  int32_t rank0[CV];
#pragma unroll
  for (int u = 0; u < CV; ++u) rank0[u] = 0;
  if (part_ties) {
    int32_t incl[CV];
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      const int64_t j0 = (v0 + (int64_t)u * CT + tid) * n;
      int32_t cnt = 0;  // (ids past the row, zeros of the buffer loads, do not count)
#pragma unroll
      for (int e = 0; e < n; ++e) cnt += j0 + e < hi && key_of<DT>(vec_elem<DT>(v[u], e)) == rs.vcut ? 1 : 0;
      incl[u] = wave_incl_scan(cnt);
      rank0[u] = incl[u] - cnt;
      if (lane == WAVE - 1) s_wt[u * NW + wid] = incl[u];
    }
    if (tid == 0) {
      int32_t before = 0;
      for (int c2 = 0; c2 < c; ++c2) before += P.rties[r * NCHK + c2];
      s_before = before;
    }
    __syncthreads();
    int32_t run = s_before;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      int32_t below = 0, tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int32_t t = s_wt[u * NW + w];
        below += w < wid ? t : 0;
        tot += t;
      }
      rank0[u] += run + below;
      run += tot;
    }
  }
  // kept: every value of an unfiltered row; a nucleus row's values above the cut key, and the
  // ones at it while their rank is below ktie (all of them at INT_MAX, none at 0).  The value
  // is dense_P's (p, over the kept mass for nucleus and renormalised rows) or, raw_p, p itself:
  // the row's choice is a branch around the loop (a select in it would divide every value).
  auto write_rows = [&](auto div_tag) {
    constexpr bool DIV = decltype(div_tag)::value;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      const int64_t j0 = (v0 + (int64_t)u * CT + tid) * n;
      if (j0 >= hi) continue;
      float x[n];
      int32_t seen = 0;
#pragma unroll
      for (int e = 0; e < n; ++e) {
        const float xe = vec_elem<DT>(v[u], e);
        const uint32_t k = key_of<DT>(xe);
        const bool tie = hist && k == rs.vcut;
        const bool kept = !hist || k > rs.vcut || (tie && (int64_t)rank0[u] + seen < (int64_t)rs.ktie);
        seen += tie ? 1 : 0;
        const float pe = prob_of(xe, T, rs.m_f, rs.invZ);
        x[e] = kept ? (DIV ? pe / rs.S_f : pe) : 0.f;
      }
      store_vec(j0, x);
    }
  };
  // raw_p with the input probabilities (logs as the rows): the kept entries copied from them
  auto copy_rows = [&]() {
    const float* srow = P.src_p + r * P.src_stride;
#pragma unroll
    for (int u = 0; u < CV; ++u) {
      const int64_t j0 = (v0 + (int64_t)u * CT + tid) * n;
      if (j0 >= hi) continue;
      float x[n];
      int32_t seen = 0;
#pragma unroll
      for (int e = 0; e < n; ++e) {
        const uint32_t k = key_of<DT>(vec_elem<DT>(v[u], e));
        const bool tie = hist && k == rs.vcut;
        const bool kept = !hist || k > rs.vcut || (tie && (int64_t)rank0[u] + seen < (int64_t)rs.ktie);
        seen += tie ? 1 : 0;
        x[e] = kept && j0 + e < hi ? srow[j0 + e] : 0.f;
      }
      store_vec(j0, x);
    }
  };
  if (P.raw_p && P.src_p)
    copy_rows();
  else if (!P.raw_p && (rs.mode == M_HIST || rs.norm))
    write_rows(std::true_type{});
  else
    write_rows(std::false_type{});
}

// ---------------------------------------------------------------------------------------
// filter_target_probs on probabilities (runtime/worker.py:473-508): each row becomes a request
// of its own at temperature 1 whose logits are log p (softmax(log p) = p / sum(p), and top-k,
// min-p and the order of the values are those of p).  One workgroup per row writes log p and
// the row's float64 mass, and the row's parameters from its request's: the top-p divided by the
// mass when the backend compares the raw mass ranked ahead with top_p (top_p_over_mass).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(CT) void k_prob_prep(const float* __restrict__ probs, int64_t pstride, int64_t V,
                                                  int32_t T, const int32_t* top_ks, const float* top_ps,
                                                  const float* min_ps, int32_t top_p_over_mass, int32_t vec4,
                                                  float* __restrict__ logs, int64_t lstride, int32_t* row_k,
                                                  float* row_p, float* row_minp, float* row_t) {
  __shared__ double sd[CT / WAVE];
  const int64_t r = blockIdx.x;
  const float* prow = probs + r * pstride;
  float* lrow = logs + r * lstride;
  double mass = 0.0;
  if (vec4) {  // rows 16-byte aligned, V a multiple of 4: four 16-byte loads in flight a thread
    constexpr int U = 4;
    const int64_t nv = V / 4;
    for (int64_t q0 = threadIdx.x; q0 < nv; q0 += (int64_t)CT * U) {
      float4 p[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + (int64_t)u * CT;
        p[u] = q < nv ? reinterpret_cast<const float4*>(prow)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + (int64_t)u * CT;
        if (q >= nv) continue;
        mass += (double)p[u].x + (double)p[u].y + (double)p[u].z + (double)p[u].w;
        reinterpret_cast<float4*>(lrow)[q] = make_float4(logf(p[u].x), logf(p[u].y), logf(p[u].z), logf(p[u].w));
      }
    }
  } else {
    for (int64_t j = threadIdx.x; j < V; j += CT) {
      const float p = prow[j];
      mass += (double)p;
      lrow[j] = logf(p);
    }
  }
  mass = block_sum<CT / WAVE>(mass, sd);
  if (threadIdx.x == 0) {
    const int64_t b = r / T;
    const float tp = top_ps ? top_ps[b] : 1.f;
    row_k[r] = top_ks[b];
    row_p[r] = top_p_over_mass && mass > 0.0 ? (float)((double)tp / mass) : tp;
    row_minp[r] = min_ps ? min_ps[b] : 0.f;
    row_t[r] = 1.f;
  }
}

// ---------------------------------------------------------------------------------------
// Greedy verify (verification/caps.py:32-59, verification/ragged.py:51-76)
// ---------------------------------------------------------------------------------------
__device__ inline int64_t chunk_argmax(const ChunkStat* cs, int C) {
  float M = -INFINITY;
  int32_t arg = INT_MAX;
  for (int c = 0; c < C; ++c)
    if (cs[c].m > M) {
      M = cs[c].m;
      arg = cs[c].arg;
    }
  return arg == INT_MAX ? 0 : arg;
}

__global__ void k_greedy_accept(const ChunkStat* cstat, int C, const int64_t* cand, const int32_t* lens,
                                int32_t cap_static, const int32_t* prefix, int32_t bs, int32_t T,
                                int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                                int32_t* new_seq, int64_t* top1_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= bs) return;
  int cap = lens ? lens[b] : cap_static;
  cap = cap < 1 ? 1 : (cap > T ? T : cap);
  int acc = cap - 1;
  for (int i = 0; i < cap - 1; ++i) {
    if (cand[(int64_t)b * T + i + 1] != chunk_argmax(cstat + ((int64_t)b * T + i) * C, C)) {
      acc = i;
      break;
    }
  }
  const int64_t bon = chunk_argmax(cstat + ((int64_t)b * T + acc) * C, C);
  for (int i = 0; i < T; ++i) {
    const int64_t proposed = i < T - 1 ? cand[(int64_t)b * T + i + 1] : 0;
    output[(int64_t)b * T + i] = i == acc ? bon : proposed;
    if (top1_out) top1_out[(int64_t)b * T + i] = chunk_argmax(cstat + ((int64_t)b * T + i) * C, C);
  }
  accept[b] = acc;
  commit[b] = acc + 1;
  bonus[b] = bon;
  new_seq[b] = prefix[b] + acc + 1;
}

// Top-k API: merge chunk candidate lists of each row (one workgroup per row).
template <int DT>
__global__ __launch_bounds__(256) void k_topk_merge(const ChunkStat* cstat, const uint64_t* cand, int C, int kcand,
                                                    int32_t K, float* values_out, int64_t* ids_out, int sort_by_id) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ uint32_t hist256[256];
  __shared__ uint64_t su[2];
  __shared__ int32_t s_cnt;
  uint64_t* buf = reinterpret_cast<uint64_t*>(dyn);
  uint64_t* top = buf + (size_t)C * kcand;
  const int64_t r = blockIdx.x;
  int n = 0;
  for (int c = 0; c < C; ++c) {
    const int nc = cstat[r * C + c].ncand;
    for (int i = threadIdx.x; i < nc; i += blockDim.x) buf[n + i] = cand[(r * C + c) * (int64_t)kcand + i];
    n += nc;
  }
  __syncthreads();
  const int kk = select_top<DT == DSV_BF16 ? 40 : 56>(buf, n, K, top, hist256, su, &s_cnt);
  for (int i = threadIdx.x; i < K; i += blockDim.x) {
    const bool ok = i < kk;
    const uint64_t v = ok ? buf[i] : 0ull;
    if (values_out) values_out[r * K + i] = ok ? value_of_key<DT>(unpack_key(v)) : -INFINITY;
    if (!sort_by_id)
      ids_out[r * K + i] = ok ? (int64_t)unpack_id(v) : -1;
    else
      top[i] = ok ? (uint64_t)unpack_id(v) : ~0ull;
  }
  if (sort_by_id) {
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
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

static int64_t align_up(int64_t x, int64_t al) { return (x + al - 1) / al * al; }

struct WsLayout {
  int64_t rowsum, lists, cstat, cand, hpart, nhist, nuc, rbonus, rties, plans, step_ok, req_cnt, deferred, pbits, total;
};
static void launch_chunk(const KParams& P, int dtype, unsigned grid, hipStream_t stream) {
  if (dtype == DSV_BF16) {
    if (P.aligned)
      hipLaunchKernelGGL((k_chunk<DSV_BF16, true>), dim3(grid), dim3(CT), 0, stream, P);
    else
      hipLaunchKernelGGL((k_chunk<DSV_BF16, false>), dim3(grid), dim3(CT), 0, stream, P);
  } else {
    if (P.aligned)
      hipLaunchKernelGGL((k_chunk<DSV_F32, true>), dim3(grid), dim3(CT), 0, stream, P);
    else
      hipLaunchKernelGGL((k_chunk<DSV_F32, false>), dim3(grid), dim3(CT), 0, stream, P);
  }
}

static int chunks_per_row(int64_t vocab, int dtype) {
  const int64_t che = dtype == DSV_BF16 ? Elems<DSV_BF16>::chunk : Elems<DSV_F32>::chunk;
  return (int)((vocab + che - 1) / che);
}
static int64_t pen_words(int64_t vocab) { return (vocab + 31) / 32; }
static WsLayout ws_layout(int64_t rows, int32_t bs, int64_t vocab, int dtype, int kcand, bool history) {
  WsLayout w;
  const int C = chunks_per_row(vocab, dtype);
  int64_t o = 0;
  auto take = [&](int64_t& field, int64_t bytes) {
    field = o;
    o = align_up(o + bytes, 256);
  };
  take(w.rowsum, rows * (int64_t)sizeof(RowSum));
  take(w.lists, rows * DSV_LIST_K * (int64_t)sizeof(ListEntry));
  take(w.cstat, rows * C * (int64_t)sizeof(ChunkStat));
  take(w.cand, rows * C * (int64_t)kcand * 8);
  take(w.hpart, kcand ? rows * C * (int64_t)(HWIN / 2) * 4 : 0);
  take(w.nhist, kcand ? (int64_t)(bs > NUC_GRID ? bs : NUC_GRID) * 65536 * 4 : 0);
  take(w.nuc, (rows + 1) * 4);
  take(w.rbonus, rows * 8);
  take(w.rties, rows * NCHK * 4);
  take(w.plans, rows * (int64_t)sizeof(DrawPlan));
  take(w.step_ok, rows * 4);
  take(w.req_cnt, (int64_t)bs * 4);
  take(w.deferred, (int64_t)bs * 4);
  take(w.pbits, history ? (int64_t)bs * pen_words(vocab) * 4 : 0);
  w.total = o;
  return w;
}

extern "C" int64_t dsv_verify_workspace_bytes(int64_t rows, int32_t bs, int32_t T, int64_t vocab) {
  (void)T;
  return ws_layout(rows, bs, vocab, DSV_F32, DSV_LIST_K, true).total;  // the largest layout
}
extern "C" int64_t dsv_greedy_workspace_bytes(int64_t rows, int64_t vocab) {
  return ws_layout(rows, 1, vocab, DSV_F32, 0, false).total;
}


// Profiling aid: events recorded around the chunk-pass launch of this thread's next verify
// calls (NULL, NULL: off).
static thread_local hipEvent_t g_prof_start = nullptr, g_prof_stop = nullptr;
extern "C" int dsv_profile_events(void* start, void* stop) {
  g_prof_start = reinterpret_cast<hipEvent_t>(start);
  g_prof_stop = reinterpret_cast<hipEvent_t>(stop);
  return DSV_OK;
}

// Validation and kernel parameters shared by the verify step and the target-distribution
// entry (drafts = false: candidates, q, uniforms and outputs may be absent).
static int verify_prepare(const dsv_verify_args& a, bool drafts, const char* what, KParams& P, bool& hist_possible) {
  if (a.logits_dtype != DSV_BF16 && a.logits_dtype != DSV_F32)
    DSV_FAIL(DSV_ERR_INVALID, "%s: logits must be float32 or bfloat16", what);
  if (a.bs <= 0 || a.T < 1 || a.vocab < 1 || a.rows < 0 || a.row_stride < a.vocab)
    DSV_FAIL(DSV_ERR_INVALID, "%s: invalid shape (bs %d, T %d, vocab %lld, rows %lld)", what, a.bs, a.T,
             (long long)a.vocab, (long long)a.rows);
  if (a.vocab >= (1ll << 31) || a.rows >= (1ll << 31))
    DSV_FAIL(DSV_ERR_INVALID, "%s: vocab and rows must be < 2^31", what);
  if (a.bs > 65535) DSV_FAIL(DSV_ERR_INVALID, "%s: at most 65535 requests per call", what);
  if (!a.row_offsets && a.rows != (int64_t)a.bs * a.T)
    DSV_FAIL(DSV_ERR_INVALID, "%s: dense layout needs rows == bs*T (%lld != %d*%d)", what, (long long)a.rows, a.bs,
             a.T);
  if (!a.logits || !a.temperatures || !a.top_ks || ((a.filter || a.sparse_joint) && !a.top_ps) || !a.workspace)
    DSV_FAIL(DSV_ERR_INVALID, "%s: required pointer is null", what);
  if (a.sparse_joint &&
      (!drafts || a.backend != DSV_BACKEND_FLASHINFER || a.need_min_p || a.any_greedy || a.max_top_k < 1 ||
       a.max_top_k > SJ_CAP || a.max_top_k > a.vocab))
    DSV_FAIL(DSV_ERR_INVALID,
             "%s: the sparse joint target needs the verify step, the flashinfer backend, no min-p, no greedy "
             "rows and 1 <= max_top_k <= %d (<= vocab)", what, SJ_CAP);
  if (drafts) {
    // (a block of one row verifies no draft: its q and per-step coins are empty arrays)
    const bool steps = a.T >= 2;
    if (!a.top_ps || !a.candidates || (steps && (!a.q_ids || !a.q_values || !a.uniforms)) || !a.uniform_final ||
        !a.prefix_lens || !a.accept || !a.commit || !a.bonus || !a.output || !a.new_seq)
      DSV_FAIL(DSV_ERR_INVALID, "%s: required pointer is null", what);
    if (a.K < 1 || a.K > QMAX) DSV_FAIL(DSV_ERR_INVALID, "%s: q width K=%d outside [1, %d]", what, a.K, QMAX);
  }
  if (a.hist_ids && a.hist_len < 0) DSV_FAIL(DSV_ERR_INVALID, "%s: negative hist_len", what);
  if (a.kv_slots && a.page_table && a.page_cols < 1) DSV_FAIL(DSV_ERR_INVALID, "%s: empty page table", what);
  if (a.backend != DSV_BACKEND_PYTORCH && a.backend != DSV_BACKEND_FLASHINFER)
    DSV_FAIL(DSV_ERR_INVALID, "%s: unknown backend %d", what, a.backend);
  hist_possible = a.filter && a.max_top_k > DSV_LIST_K;
  const int C = chunks_per_row(a.vocab, a.logits_dtype);
  if (C > NCHK)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "%s: vocab %lld needs %d chunks (> %d)", what, (long long)a.vocab, C, NCHK);
  const bool history = a.hist_ids && a.hist_len > 0;
  const WsLayout w = ws_layout(a.rows, a.bs, a.vocab, a.logits_dtype, DSV_LIST_K, history);
  if (a.workspace_bytes < w.total)
    DSV_FAIL(DSV_ERR_WORKSPACE, "%s: workspace %lld < %lld bytes", what, (long long)a.workspace_bytes,
             (long long)w.total);
  const size_t esize = a.logits_dtype == DSV_BF16 ? 2 : 4;
  memset(&P, 0, sizeof(P));
  P.a = a;
  if (!history) P.a.hist_ids = nullptr;
  char* ws = reinterpret_cast<char*>(a.workspace);
  P.rowsum = reinterpret_cast<RowSum*>(ws + w.rowsum);
  P.lists = reinterpret_cast<ListEntry*>(ws + w.lists);
  P.cstat = reinterpret_cast<ChunkStat*>(ws + w.cstat);
  P.cand = reinterpret_cast<uint64_t*>(ws + w.cand);
  P.hpart = reinterpret_cast<uint32_t*>(ws + w.hpart);
  P.nhist = reinterpret_cast<uint32_t*>(ws + w.nhist);
  P.nuc_rows = reinterpret_cast<int32_t*>(ws + w.nuc);
  P.rbonus = reinterpret_cast<int64_t*>(ws + w.rbonus);
  P.rties = reinterpret_cast<int32_t*>(ws + w.rties);
  P.plans = reinterpret_cast<DrawPlan*>(ws + w.plans);
  P.req_cnt = reinterpret_cast<uint32_t*>(ws + w.req_cnt);
  P.deferred = reinterpret_cast<uint32_t*>(ws + w.deferred);
  P.step_ok = reinterpret_cast<int32_t*>(ws + w.step_ok);
  P.pbits = history ? reinterpret_cast<uint32_t*>(ws + w.pbits) : nullptr;
  P.pwords = pen_words(a.vocab);
  P.C = C;
  P.kcand = DSV_LIST_K;
  P.aligned = ((uintptr_t)a.logits % 16 == 0) && ((a.row_stride * (int64_t)esize) % 16 == 0) &&
              a.vocab * (int64_t)esize >= 16;
  P.softmax = 1;
  return DSV_OK;
}

// The row stage: history bitmaps, the chunk pass, the row merge, and the full-histogram rows.
static int launch_rows(const KParams& P, bool hist_possible, bool profile, hipStream_t stream) {
  const dsv_verify_args& a = P.a;
  if (profile && g_prof_start && g_prof_stop && hipEventRecord(g_prof_start, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_verify: cannot record the profiling start event");
  launch_chunk(P, a.logits_dtype, (unsigned)(a.rows * P.C), stream);
  if (profile && g_prof_start && g_prof_stop && hipEventRecord(g_prof_stop, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_verify: cannot record the profiling stop event");
  if (a.logits_dtype == DSV_BF16) {
    if (P.aligned)
      hipLaunchKernelGGL((k_merge<DSV_BF16, true>), dim3((unsigned)a.rows), dim3(CT), 0, stream, P);
    else
      hipLaunchKernelGGL((k_merge<DSV_BF16, false>), dim3((unsigned)a.rows), dim3(CT), 0, stream, P);
  } else {
    if (P.aligned)
      hipLaunchKernelGGL((k_merge<DSV_F32, true>), dim3((unsigned)a.rows), dim3(CT), 0, stream, P);
    else
      hipLaunchKernelGGL((k_merge<DSV_F32, false>), dim3((unsigned)a.rows), dim3(CT), 0, stream, P);
  }
  DSV_CHECK_LAUNCH("k_chunk / k_merge");
  if (hist_possible && !P.final_nuc) {  // rows the merge listed: the full histogram (bf16) or radix descent (fp32)
    // (bf16 workgroups each own a global histogram area; fp32 ones work in LDS alone, one per CU)
    const int cap = a.logits_dtype == DSV_BF16 ? NUC_GRID : NUC_GRID_F32;
    const int grid = (int)(a.rows < cap ? a.rows : cap);
    if (a.logits_dtype == DSV_BF16) {
      const size_t nuc_lds = (size_t)HIST_WORDS * 4;
      if (P.aligned) {
        (void)hipFuncSetAttribute((const void*)k_nuc<DSV_BF16, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)nuc_lds);
        hipLaunchKernelGGL((k_nuc<DSV_BF16, true>), dim3(grid), dim3(NUC_THREADS), nuc_lds, stream, P);
      } else {
        (void)hipFuncSetAttribute((const void*)k_nuc<DSV_BF16, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)nuc_lds);
        hipLaunchKernelGGL((k_nuc<DSV_BF16, false>), dim3(grid), dim3(NUC_THREADS), nuc_lds, stream, P);
      }
    } else {
      const size_t nuc_lds = sizeof(F32NucLds);
      if (P.aligned) {
        (void)hipFuncSetAttribute((const void*)k_nuc<DSV_F32, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)nuc_lds);
        hipLaunchKernelGGL((k_nuc<DSV_F32, true>), dim3(grid), dim3(NUC_THREADS), nuc_lds, stream, P);
      } else {
        (void)hipFuncSetAttribute((const void*)k_nuc<DSV_F32, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)nuc_lds);
        hipLaunchKernelGGL((k_nuc<DSV_F32, false>), dim3(grid), dim3(NUC_THREADS), nuc_lds, stream, P);
      }
    }
    DSV_CHECK_LAUNCH("k_nuc");
  }
  return DSV_OK;
}

extern "C" int dsv_verify(const dsv_verify_args* args, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "dsv_verify: null arguments");
  const dsv_verify_args& a = *args;
  KParams P;
  bool hist_possible = false;
  const int rc = verify_prepare(a, true, "dsv_verify", P, hist_possible);
  if (rc != DSV_OK) return rc;
  if (a.rows == 0) return DSV_OK;
  const int stages = a.stages ? a.stages : 7;
  // with k_final in the launch, each request's workgroup resolves its own full-histogram rows
  // (usually none: the merge's windows settle the cut) and no k_nuc launch is needed
  P.final_nuc = (stages & 4) && hist_possible ? 1 : 0;
  // The row merge writes the outputs of the requests whose accepted row drew its token there
  // (greedy and support-list rows).  k_final takes the rest: requests whose accepted row is a
  // dense row (unfiltered or nucleus: only when a top-k above the support list, or no filter,
  // can occur), and requests whose ragged row offsets leave rows outside the logits.
  const bool all_greedy = a.any_greedy && a.max_top_k <= 1;
  const bool dense_possible = !all_greedy && (!a.filter || a.max_top_k > DSV_LIST_K || a.sparse_joint);
  P.only_deferred = (stages & 1) ? 1 : 0;
  if (stages & 1) {
    const int rc2 = launch_rows(P, hist_possible, true, stream);
    if (rc2 != DSV_OK) return rc2;
  }
  if ((stages & 4) && (!(stages & 1) || dense_possible || a.row_offsets)) {
    const size_t lds = !P.final_nuc ? 0 : a.logits_dtype == DSV_BF16 ? (size_t)HIST_WORDS * 4 : sizeof(F32NucLds);
    auto go = [&](const void* fn, auto kernel) {
      if (lds) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      hipLaunchKernelGGL(kernel, dim3((unsigned)a.bs * KF_ROLES), dim3(FCT), lds, stream, P);
    };
    if (a.logits_dtype == DSV_BF16) {
      if (P.aligned)
        go((const void*)k_final<DSV_BF16, true>, k_final<DSV_BF16, true>);
      else
        go((const void*)k_final<DSV_BF16, false>, k_final<DSV_BF16, false>);
    } else {
      if (P.aligned)
        go((const void*)k_final<DSV_F32, true>, k_final<DSV_F32, true>);
      else
        go((const void*)k_final<DSV_F32, false>, k_final<DSV_F32, false>);
    }
    DSV_CHECK_LAUNCH("k_final");
  }
  return DSV_OK;
}

// The target-distribution entries: the chunk pass, the row merge, the full-histogram rows, then
// P of every (row, chunk).
static int launch_target(KParams& P, bool hist_possible, float* out, int64_t out_stride, hipStream_t stream) {
  const dsv_verify_args& a = P.a;
  const int rc = launch_rows(P, hist_possible, false, stream);
  if (rc != DSV_OK) return rc;
  const dim3 grid((unsigned)(a.rows * P.C));
  if (a.logits_dtype == DSV_BF16) {
    if (P.aligned)
      hipLaunchKernelGGL((k_dense_p<DSV_BF16, true>), grid, dim3(CT), 0, stream, P, out, out_stride);
    else
      hipLaunchKernelGGL((k_dense_p<DSV_BF16, false>), grid, dim3(CT), 0, stream, P, out, out_stride);
  } else {
    if (P.aligned)
      hipLaunchKernelGGL((k_dense_p<DSV_F32, true>), grid, dim3(CT), 0, stream, P, out, out_stride);
    else
      hipLaunchKernelGGL((k_dense_p<DSV_F32, false>), grid, dim3(CT), 0, stream, P, out, out_stride);
  }
  DSV_CHECK_LAUNCH("k_dense_p");
  return DSV_OK;
}

extern "C" int dsv_target_probs(const dsv_verify_args* args, float* out, int64_t out_stride, int32_t normalize,
                                dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "dsv_target_probs: null arguments");
  dsv_verify_args a = *args;
  a.candidates = nullptr;  // no drafts: no accept decisions, no bonus draw
  if (!out || out_stride < a.vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_target_probs: output [rows, vocab] required");
  KParams P;
  bool hist_possible = false;
  const int rc = verify_prepare(a, false, "dsv_target_probs", P, hist_possible);
  if (rc != DSV_OK) return rc;
  P.raw_p = normalize ? 0 : 1;
  if (a.rows == 0) return DSV_OK;
  return launch_target(P, hist_possible, out, out_stride, stream);
}

// the log rows' stride (floats), and the layout of the filter workspace: log p, the rows'
// parameters, then the row kernels' workspace with each row a request of its own
static int64_t filter_log_stride(int64_t vocab) { return align_up(vocab, 64); }
static int64_t filter_head_bytes(int64_t rows, int64_t vocab) {
  return align_up(rows * filter_log_stride(vocab) * 4, 256) + 4 * align_up(rows * 4, 256);
}
extern "C" int64_t dsv_filter_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows < 0 || vocab < 1) return -1;
  return filter_head_bytes(rows, vocab) + dsv_verify_workspace_bytes(rows, (int32_t)(rows > 0 ? rows : 1), 1, vocab);
}

extern "C" int dsv_filter_probs(const dsv_verify_args* args, const float* probs, int64_t probs_stride, float* out,
                                int64_t out_stride, int32_t normalize, int32_t top_p_over_mass,
                                dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (!args) DSV_FAIL(DSV_ERR_INVALID, "dsv_filter_probs: null arguments");
  const dsv_verify_args& a = *args;
  if (!probs || !out || probs_stride < a.vocab || out_stride < a.vocab)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_filter_probs: probabilities and output [rows, vocab] required");
  if (a.bs <= 0 || a.T < 1 || a.vocab < 1 || a.rows != (int64_t)a.bs * a.T || a.row_offsets)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_filter_probs: rows must be bs * T whole requests (rows %lld, bs %d, T %d)",
             (long long)a.rows, a.bs, a.T);
  if (!a.filter) DSV_FAIL(DSV_ERR_INVALID, "dsv_filter_probs: no filter flag (the input is the result)");
  if (!a.top_ks || !a.workspace) DSV_FAIL(DSV_ERR_INVALID, "dsv_filter_probs: required pointer is null");
  if (a.rows > 65535)
    DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_filter_probs: at most 65535 rows per call (%lld)", (long long)a.rows);
  const int64_t need = dsv_filter_workspace_bytes(a.rows, a.vocab);
  if (a.workspace_bytes < need)
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_filter_probs: workspace %lld < %lld bytes", (long long)a.workspace_bytes,
             (long long)need);
  const int64_t rows = a.rows, lstride = filter_log_stride(a.vocab);
  char* ws = reinterpret_cast<char*>(a.workspace);
  float* logs = reinterpret_cast<float*>(ws);
  char* prm = ws + align_up(rows * lstride * 4, 256);
  const int64_t pb = align_up(rows * 4, 256);
  int32_t* row_k = reinterpret_cast<int32_t*>(prm);
  float* row_p = reinterpret_cast<float*>(prm + pb);
  float* row_minp = reinterpret_cast<float*>(prm + 2 * pb);
  float* row_t = reinterpret_cast<float*>(prm + 3 * pb);
  const int32_t vec4 = (uintptr_t)probs % 16 == 0 && probs_stride % 4 == 0 && a.vocab % 4 == 0;
  hipLaunchKernelGGL(k_prob_prep, dim3((unsigned)rows), dim3(CT), 0, stream, probs, probs_stride, a.vocab, a.T,
                     a.top_ks, a.top_ps, a.min_ps, top_p_over_mass, vec4, logs, lstride, row_k, row_p, row_minp,
                     row_t);
  DSV_CHECK_LAUNCH("k_prob_prep");
  // each row a request at temperature 1, no penalties, no drafts
  dsv_verify_args r = a;
  r.logits = logs;
  r.logits_dtype = DSV_F32;
  r.row_stride = lstride;
  r.bs = (int32_t)rows;
  r.T = 1;
  r.verify_lens = nullptr;  // every row is filtered
  r.temperatures = row_t;
  r.top_ks = row_k;
  r.top_ps = row_p;
  r.min_ps = a.min_ps ? row_minp : nullptr;
  r.any_greedy = 0;
  r.sparse_joint = 0;
  r.hist_ids = nullptr;
  r.hist_len = 0;
  r.presence = nullptr;
  r.repetition = nullptr;
  r.candidates = nullptr;
  r.workspace = ws + filter_head_bytes(rows, a.vocab);
  r.workspace_bytes = a.workspace_bytes - filter_head_bytes(rows, a.vocab);
  KParams P;
  bool hist_possible = false;
  const int rc = verify_prepare(r, false, "dsv_filter_probs", P, hist_possible);
  if (rc != DSV_OK) return rc;
  P.raw_p = normalize ? 0 : 1;
  P.src_p = normalize ? nullptr : probs;
  P.src_stride = probs_stride;
  return launch_target(P, hist_possible, out, out_stride, stream);
}

// Argument checks shared by the greedy-verify entry points (what: the entry point's name).
static int greedy_check(const char* what, const void* logits, int32_t dtype, int64_t rows, int64_t vocab,
                        int64_t row_stride, int32_t bs, int32_t T, const int64_t* candidates,
                        const int32_t* verify_lens, int32_t cap, const int32_t* prefix_lens, int32_t* accept,
                        int32_t* commit, int64_t* bonus, int64_t* output, int32_t* new_seq) {
  if (dtype != DSV_BF16 && dtype != DSV_F32) DSV_FAIL(DSV_ERR_INVALID, "%s: logits must be float32 or bfloat16", what);
  if (bs <= 0 || T < 1 || vocab < 1 || row_stride < vocab || rows != (int64_t)bs * T)
    DSV_FAIL(DSV_ERR_INVALID, "%s: logits must be [bs*T, V] (rows %lld, bs %d, T %d)", what, (long long)rows, bs, T);
  if (vocab >= (1ll << 31) || rows >= (1ll << 31)) DSV_FAIL(DSV_ERR_INVALID, "%s: vocab and rows must be < 2^31", what);
  if (!verify_lens && (cap < 1 || cap > T)) DSV_FAIL(DSV_ERR_INVALID, "%s: cap %d outside [1, %d]", what, cap, T);
  if (!logits || !candidates || !prefix_lens || !accept || !commit || !bonus || !output || !new_seq)
    DSV_FAIL(DSV_ERR_INVALID, "%s: required pointer is null", what);
  return DSV_OK;
}

// The greedy verify's two launches: the chunk pass (per-chunk max / first argmax into
// cstat[rows * C], every entry written) and the per-request acceptance reading them.
static int greedy_launch(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                         int32_t bs, int32_t T, const int64_t* candidates, const int32_t* verify_lens, int32_t cap,
                         const int32_t* prefix_lens, int32_t* accept, int32_t* commit, int64_t* bonus,
                         int64_t* output, int32_t* new_seq, int64_t* top1_out, ChunkStat* cstat,
                         hipStream_t stream) {
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
  P.a.candidates = candidates;
  P.cstat = cstat;
  P.C = chunks_per_row(vocab, dtype);
  P.aligned = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esize) % 16 == 0) &&
              vocab * (int64_t)esize >= 16;
  P.force_greedy = 1;
  const bool prof = g_prof_start && g_prof_stop;
  if (prof && hipEventRecord(g_prof_start, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_greedy_verify: cannot record the profiling start event");
  launch_chunk(P, dtype, (unsigned)(rows * P.C), stream);
  if (prof && hipEventRecord(g_prof_stop, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_greedy_verify: cannot record the profiling stop event");
  DSV_CHECK_LAUNCH("k_chunk");
  hipLaunchKernelGGL(k_greedy_accept, dim3((bs + 63) / 64), dim3(64), 0, stream, P.cstat, P.C, candidates,
                     verify_lens, cap, prefix_lens, bs, T, accept, commit, bonus, output, new_seq, top1_out);
  DSV_CHECK_LAUNCH("k_greedy_accept");
  return DSV_OK;
}

extern "C" int dsv_greedy_verify(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                                 int32_t bs, int32_t T, const int64_t* candidates, const int32_t* verify_lens,
                                 int32_t cap, const int32_t* prefix_lens, int32_t* accept, int32_t* commit,
                                 int64_t* bonus, int64_t* output, int32_t* new_seq, int64_t* top1_out,
                                 void* workspace, int64_t workspace_bytes, dsv_stream_t stream_) {
  const int rc = greedy_check("dsv_greedy_verify", logits, dtype, rows, vocab, row_stride, bs, T, candidates,
                              verify_lens, cap, prefix_lens, accept, commit, bonus, output, new_seq);
  if (rc != DSV_OK) return rc;
  if (!workspace) DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify: required pointer is null");
  const WsLayout w = ws_layout(rows, 1, vocab, dtype, 0, false);
  if (workspace_bytes < w.total)
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_greedy_verify: workspace %lld < %lld", (long long)workspace_bytes,
             (long long)w.total);
  ChunkStat* cstat = reinterpret_cast<ChunkStat*>(reinterpret_cast<char*>(workspace) + w.cstat);
  return greedy_launch(logits, dtype, rows, vocab, row_stride, bs, T, candidates, verify_lens, cap, prefix_lens,
                       accept, commit, bonus, output, new_seq, top1_out, cstat,
                       reinterpret_cast<hipStream_t>(stream_));
}

// ---------------------------------------------------------------------------------------
// Allocation-free greedy verify: the per-chunk statistics go to a static device array instead
// of a caller workspace.  Each device holds its own copy for the life of the process; its
// address is looked up once per device (hipGetSymbolAddress, the device current) and only that
// address is handed to kernels -- the array's name in host code is not a device address.
// ---------------------------------------------------------------------------------------
constexpr int64_t NOALLOC_CHUNK_STATS = 65536;  // (row, chunk) statistics: 65536 x 40 B = 2.5 MiB
constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) ChunkStat scratch[NOALLOC_CHUNK_STATS];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// The scratch address on the current device (looked up on the first call there).
static int noalloc_scratch(hipStream_t stream, ChunkStat** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_greedy_verify_noalloc: no usable current device");
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess)
      DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify_noalloc: cannot query the stream's device");
    if (sdev != dev)
      DSV_FAIL(DSV_ERR_INVALID, "dsv_greedy_verify_noalloc: the stream belongs to device %d, device %d is current",
               (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      DSV_FAIL(DSV_ERR_LAUNCH, "dsv_greedy_verify_noalloc: scratch address lookup failed on device %d: %s", dev,
               hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = reinterpret_cast<ChunkStat*>(g_scratch_ptr[dev]);
  return DSV_OK;
}

extern "C" int dsv_greedy_verify_noalloc(const void* logits, int32_t dtype, int64_t rows, int64_t vocab,
                                         int64_t row_stride, int32_t bs, int32_t T, const int64_t* candidates,
                                         const int32_t* verify_lens, int32_t cap, const int32_t* prefix_lens,
                                         int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                                         int32_t* new_seq, int64_t* top1_out, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int rc = greedy_check("dsv_greedy_verify_noalloc", logits, dtype, rows, vocab, row_stride, bs, T,
                              candidates, verify_lens, cap, prefix_lens, accept, commit, bonus, output, new_seq);
  if (rc != DSV_OK) return rc;
  const int64_t need = rows * chunks_per_row(vocab, dtype);
  if (need > NOALLOC_CHUNK_STATS)
    DSV_FAIL(DSV_ERR_INVALID,
             "dsv_greedy_verify_noalloc: %lld rows x %d chunks exceed the %lld chunk statistics of the static "
             "scratch (use dsv_greedy_verify with a workspace)",
             (long long)rows, chunks_per_row(vocab, dtype), (long long)NOALLOC_CHUNK_STATS);
  ChunkStat* cstat = nullptr;
  const int rc2 = noalloc_scratch(stream, &cstat);
  if (rc2 != DSV_OK) return rc2;
  // every (row, chunk) statistic is written by the chunk pass before the acceptance reads it:
  // nothing in the scratch needs clearing
  return greedy_launch(logits, dtype, rows, vocab, row_stride, bs, T, candidates, verify_lens, cap, prefix_lens,
                       accept, commit, bonus, output, new_seq, top1_out, cstat, stream);
}

extern "C" int64_t dsv_topk_workspace_bytes(int64_t rows, int64_t vocab, int32_t k) {
  const int C = chunks_per_row(vocab, DSV_F32);
  return align_up((int64_t)rows * C * ((int64_t)sizeof(ChunkStat) + (int64_t)k * 8), 256);
}

extern "C" int dsv_topk(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride, int32_t k,
                        float* values_out, int64_t* ids_out, int32_t sort_by_id, void* workspace,
                        int64_t workspace_bytes, dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (dtype != DSV_BF16 && dtype != DSV_F32) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: logits must be float32 or bfloat16");
  if (rows < 0 || vocab < 1 || row_stride < vocab) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: invalid shape");
  if (vocab >= (1ll << 31) || rows >= (1ll << 31)) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: vocab and rows must be < 2^31");
  if (k < 1 || k > TOPK_MAX || k > vocab)
    DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: k=%d outside [1, min(%d, V)]", k, TOPK_MAX);
  if (!logits || !ids_out || !workspace) DSV_FAIL(DSV_ERR_INVALID, "dsv_topk: null pointer");
  if (rows == 0) return DSV_OK;
  const int C = chunks_per_row(vocab, dtype);
  const size_t merge_lds = ((size_t)C * k + k) * 8;
  if (merge_lds > 150 * 1024) DSV_FAIL(DSV_ERR_UNSUPPORTED, "dsv_topk: k=%d with %d chunks needs too much LDS", k, C);
  if (workspace_bytes < dsv_topk_workspace_bytes(rows, vocab, k))
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_topk: workspace too small");
  const size_t esize = dtype == DSV_BF16 ? 2 : 4;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.a.logits = logits;
  P.a.logits_dtype = dtype;
  P.a.rows = rows;
  P.a.vocab = vocab;
  P.a.row_stride = row_stride;
  P.cstat = reinterpret_cast<ChunkStat*>(workspace);
  P.cand = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + (size_t)rows * C * sizeof(ChunkStat));
  P.C = C;
  P.kcand = k;
  P.aligned = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esize) % 16 == 0) &&
              vocab * (int64_t)esize >= 16;
  if (g_prof_start && g_prof_stop && hipEventRecord(g_prof_start, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_topk: cannot record the profiling start event");
  launch_chunk(P, dtype, (unsigned)(rows * C), stream);
  if (g_prof_start && g_prof_stop && hipEventRecord(g_prof_stop, stream) != hipSuccess)
    DSV_FAIL(DSV_ERR_LAUNCH, "dsv_topk: cannot record the profiling stop event");
  if (dtype == DSV_BF16) {
    (void)hipFuncSetAttribute((const void*)k_topk_merge<DSV_BF16>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)merge_lds);
    hipLaunchKernelGGL(k_topk_merge<DSV_BF16>, dim3((unsigned)rows), dim3(256), merge_lds, stream, P.cstat, P.cand, C,
                       k, k, values_out, ids_out, sort_by_id);
  } else {
    (void)hipFuncSetAttribute((const void*)k_topk_merge<DSV_F32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)merge_lds);
    hipLaunchKernelGGL(k_topk_merge<DSV_F32>, dim3((unsigned)rows), dim3(256), merge_lds, stream, P.cstat, P.cand, C,
                       k, k, values_out, ids_out, sort_by_id);
  }
  DSV_CHECK_LAUNCH("dsv_topk");
  return DSV_OK;
}
