/*
 * dspine_verify.h -- C ABI of the MI355X (gfx950) draft-verification library.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, launches on that
 * stream without any host synchronisation or device allocation, and returns DSV_OK (0) or an
 * error code; dsv_last_error() describes the last failure of the calling thread.  Contract
 * violations are detected before any launch (DSV_ERR_INVALID), so a caller can map them to
 * ValueError exactly as the reference does before its Triton launches.
 *
 * Reference interfaces replaced (paths relative to the reference's package sglang_dspine):
 *   dsv_verify            sampling/target.py:34-122 (TargetDistribution.sample_prefix), which
 *                         builds P (runtime/worker.py:440-508) and runs
 *                         sampling/sparse/accept.py:463-543 (accept_sparse); also
 *                         runtime/worker.py:1048-1089 (_dspine_verify) and
 *                         runtime/worker.py:511-581 (dspine_accept_sampling)
 *   dsv_greedy_verify     verification/caps.py:331-379 (greedy branch + _accept_capped :32-59)
 *                         and verification/ragged.py:282-335 (greedy branch + _accept :51-76)
 *   dsv_topk              kernels/dspine.py:165-207 (topk_ids) and the tie rule of
 *                         layers/fp8/coarse.py:19-34 / sampling/tp_head.py:9-14
 *   dsv_uniforms          sampling/random.py:71-91 (seeded_uniforms / _uniforms :46-68)
 *   dsv_adjust_logits     sampling/compact.py:14-79 (adjust_logits: the additive and the scaling
 *                         operation, compact.py:32-45)
 *   dsv_adjust_history    sampling/compact.py:47-63 with SGLang's presence/repetition penalizers
 *                         given as a per-request token history
 *   dsv_logits_padding    sampling/padding.py:4-12 (logits_padding)
 *   dsv_target_probs      runtime/worker.py:440-470 (build_dspine_target_probs)
 *   dsv_filter_probs      runtime/worker.py:473-508 (filter_target_probs, its backend filter
 *                         :52-67 on given probabilities)
 *   dsv_accept_chain      sampling/rejection.py:12-153 (_sample_capped_chain,
 *                         sample_capped_chain_from_probs) and sampling/sparse/accept.py:81-543
 *                         (accept_sparse with dense, RAW or packed P)
 *   dsv_compress          sampling/sparse/accept.py:7-78,422-460 (compress_probs)
 *   dsv_pack_joint        sampling/sparse/target.py:22-66,95-178 (_pack_joint, _overflow_dense,
 *                         build_sparse_target)
 *   dsv_sample_chain      kernels/dspine.py:616-772 (serial_sample_chain)
 *   dsv_rs_table          kernels/dspine.py:505-613 (serial_rs_table)
 *   dsv_factor_table      sampling/factorized/kernels.py:179-300 (factor_table) with
 *                         sampling/factorized/cancellation.py:82-147 (apply_direct_fallback);
 *                         dsv_factor_widen / dsv_factor_gemm: weights.py:34-80 (build_cache)
 *   dsv_window_index      verification/sps.py:27-32,87-98 (_indices)
 *   dsv_sps_plan          verification/sps.py:35-58 (allocate_verify_lens) and :61-99
 *                         (device_plan: lengths, layout row pointer, _indices)
 *   dsv_commit_accept     the commit after the accept buffers (SGLang's _commit_accept, not in
 *                         the reference; its accept-buffer discipline tests/test_tp_accept.py
 *                         :106-180)
 */
#ifndef DSPINE_VERIFY_H
#define DSPINE_VERIFY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dsv_stream_t; /* == hipStream_t */

enum {
  DSV_OK = 0,
  DSV_ERR_INVALID = 1,     /* shape / dtype / pointer contract violated (nothing launched) */
  DSV_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
  DSV_ERR_LAUNCH = 3,      /* HIP launch failure */
  DSV_ERR_WORKSPACE = 4    /* workspace too small */
};

enum { DSV_F32 = 0, DSV_BF16 = 1, DSV_F16 = 2 };

/* Sampling-backend semantics of the target filter (runtime/worker.py:482-505). */
enum {
  DSV_BACKEND_PYTORCH = 0,   /* sort, cumsum, zero rank>=k, zero (S_j - p_j) > top_p, min-p */
  DSV_BACKEND_FLASHINFER = 1 /* joint top-k / top-p support; sequential branch with min-p */
};

/* Largest top-k kept as an explicit candidate list; larger top-k use the value histogram. */
#define DSV_LIST_K 64

const char* dsv_last_error(void);
int dsv_device_count(void);

/* ---------------------------------------------------------------------------------------- */
/* Full sampled verify step: logit adjustments -> target distribution -> chain rejection with */
/* sparse q -> residual resample -> accepted-prefix compaction -> KV slot gather.            */
/* ---------------------------------------------------------------------------------------- */
typedef struct dsv_verify_args {
  /* target logits [rows, vocab], row stride in elements */
  const void* logits;
  int32_t logits_dtype; /* DSV_F32 / DSV_BF16 */
  int32_t stages;       /* 0 = whole step; else bit 0 rows, bit 1 chunk scan, bit 2 finalize */
  int64_t rows, vocab, row_stride;
  /* request layout: row(b, s) = b*T + s, or row_offsets[b] + s when row_offsets != NULL */
  int32_t bs, T;                 /* candidates [bs, T]; q rows [bs, T-1, K] */
  const int32_t* verify_lens;    /* [bs] in [1, T], NULL = T for every request */
  const void* row_offsets;       /* [bs] int32 or int64, NULL = dense layout */
  int32_t row_offsets_i64;
  /* per-request sampling parameters */
  int32_t backend;               /* DSV_BACKEND_* */
  const float* temperatures;     /* [bs] (> 0) */
  const int32_t* top_ks;         /* [bs], >= 2^30 means off */
  const float* top_ps;           /* [bs] */
  const float* min_ps;           /* [bs] or NULL */
  int32_t filter;                /* need_top_k || need_top_p || need_min_p (batch flags) */
  int32_t need_min_p;
  int32_t any_greedy;            /* rows of requests with top_k <= 1 are one-hot at argmax */
  int32_t max_top_k;             /* host-known bound on top_ks (SamplingBatchInfo.max_top_k) */
  /* 1: the reference's sparse joint target (sampling/sparse/target.py:95-178), the route        */
  /* TargetDistribution.sample_prefix takes for flashinfer batches build_sparse_target accepts   */
  /* (sampling/target.py:53-66): keep every p >= the k-th largest p (all its ties) whose         */
  /* strictly larger p hold less than top_p; a row keeping more than 32 becomes a dense row of    */
  /* every p >= the k-th.  Requires the flashinfer backend, no min-p, no greedy rows and         */
  /* 1 <= max_top_k <= 32 (the filter applies whatever the need_* flags).  dsv_verify only.      */
  int32_t sparse_joint;
  int32_t pad0;
  /* optional presence / repetition penalty over a token history [bs, hist_len] (-1 = pad) */
  const int32_t* hist_ids;
  int32_t hist_len, pad1;
  const float* presence;         /* [bs]: additive -presence on history tokens */
  const float* repetition;       /* [bs]: x<0 ? x*r : x/r on history tokens */
  /* draft proposal */
  const int64_t* candidates;     /* [bs, T]: anchor then T-1 drafts */
  const void* q_ids;             /* [bs, T-1, K] int32 or int64 (may be NULL when T == 1) */
  int32_t q_ids_i64, K;
  const float* q_values;         /* [bs, T-1, K] (may be NULL when T == 1) */
  const float* uniforms;         /* [bs, T-1] (may be NULL when T == 1) */
  const float* uniform_final;    /* [bs] */
  const int32_t* prefix_lens;    /* [bs] */
  const int32_t* page_table;     /* [bs, page_cols] (page size 1) or NULL */
  int64_t page_stride, page_cols;
  /* outputs (caller-owned) */
  int32_t* accept;               /* [bs] */
  int32_t* commit;               /* [bs] */
  int64_t* bonus;                /* [bs] */
  int64_t* output;               /* [bs, T] */
  int32_t* new_seq;              /* [bs] */
  int32_t* kv_slots;             /* [bs, T] or NULL */
  /* scratch (caller-owned device memory of dsv_verify_workspace_bytes) */
  void* workspace;
  int64_t workspace_bytes;
} dsv_verify_args;

int64_t dsv_verify_workspace_bytes(int64_t rows, int32_t bs, int32_t T, int64_t vocab);
int dsv_verify(const dsv_verify_args* args, dsv_stream_t stream);

/* Profiling aid with no counterpart in the reference: the calling thread's later dsv_verify,  */
/* dsv_greedy_verify and dsv_topk calls record `start` / `stop` (hipEvent_t, timing enabled)   */
/* on their stream right before and after the chunk-pass kernel, so a benchmark can time that */
/* kernel alone.                                                                               */
/* NULL, NULL: off.                                                                            */
int dsv_profile_events(void* start, void* stop);

/* Greedy verify (argmax acceptance): top1 = first argmax of each row, a = first mismatch   */
/* below verify_lens[b]-1 (or cap-1), bonus = top1[a]; output keeps proposals after a.      */
/* Rows are b*T + s (the full-width envelope).  top1_out [rows] (int64) is optional.        */
int dsv_greedy_verify(const void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab,
                      int64_t row_stride, int32_t bs, int32_t T, const int64_t* candidates,
                      const int32_t* verify_lens, int32_t cap, const int32_t* prefix_lens,
                      int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                      int32_t* new_seq, int64_t* top1_out, void* workspace,
                      int64_t workspace_bytes, dsv_stream_t stream);
int64_t dsv_greedy_workspace_bytes(int64_t rows, int64_t vocab);

/* dsv_greedy_verify without a workspace argument and without any allocation.  No counterpart */
/* in the reference: it is for callers that cannot allocate device memory (code under HIP      */
/* graph capture, serving loops or harnesses that forbid hipMalloc).  The per-chunk statistics */
/* live in a static device array of the library (2.5 MiB a device, held until the process     */
/* ends): rows * ceil(vocab / 20480) (bf16) or rows * ceil(vocab / 12288) (float32) must not   */
/* exceed 65536 (DSV_ERR_INVALID otherwise; e.g. 8192 bf16 rows of 151936).  Calls that        */
/* overlap on one device share that array and race; the stream must belong to the current     */
/* device.  Same arguments and outputs as dsv_greedy_verify otherwise.                         */
int dsv_greedy_verify_noalloc(const void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab,
                              int64_t row_stride, int32_t bs, int32_t T, const int64_t* candidates,
                              const int32_t* verify_lens, int32_t cap, const int32_t* prefix_lens,
                              int32_t* accept, int32_t* commit, int64_t* bonus, int64_t* output,
                              int32_t* new_seq, int64_t* top1_out, dsv_stream_t stream);

/* Top-k per row in (value desc, id asc) order, k in [1, 256].  values_out [rows, k] float32 */
/* (may be NULL), ids_out [rows, k] int64; sort_by_id != 0 re-sorts each row's ids ascending */
/* (topk_ids).  workspace: dsv_topk_workspace_bytes(rows, vocab, k) bytes of device memory.  */
int dsv_topk(const void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab,
             int64_t row_stride, int32_t k, float* values_out, int64_t* ids_out,
             int32_t sort_by_id, void* workspace, int64_t workspace_bytes, dsv_stream_t stream);
int64_t dsv_topk_workspace_bytes(int64_t rows, int64_t vocab, int32_t k);

/* Seeded uniforms [n, width] of draw stream `stream` (0..3), murmur3 keyed by              */
/* (seed, position, column).                                                                */
int dsv_uniforms(const int64_t* seeds, const void* positions, int32_t positions_i64, int64_t n,
                 int32_t width, int32_t stream_id, float* out, dsv_stream_t stream);

/* ---------------------------------------------------------------------------------------- */
/* In-place logit adjustments (one operation a call, in the caller's order, each rounded to  */
/* the logits dtype like the reference's in-place tensor ops).  Row r belongs to request     */
/* row_to_request[r] (int64) when given, else r / rows_per_request.                          */
/* ---------------------------------------------------------------------------------------- */
enum {
  DSV_ADJ_ADD = 0,  /* x += v[req, j]                      (compact.py:38-42, :56-63, :77-79) */
  DSV_ADJ_SCALE = 1 /* x = x < 0 ? x * v[req, j] : x / v   (compact.py:32-34, :43-45)        */
};
int dsv_adjust_logits(void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                      const int64_t* row_to_request, int32_t rows_per_request, int64_t requests, int32_t op,
                      const float* values, int64_t values_stride, dsv_stream_t stream);
/* Presence (x -= presence[req]) then repetition (x < 0 ? x*r : x/r) on each token of the    */
/* request's history [requests, hist_len] (int32, each token once), in place.                */
int dsv_adjust_history(void* logits, int32_t logits_dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                       const int64_t* row_to_request, int32_t rows_per_request, int64_t requests,
                       const int32_t* hist_ids, int32_t hist_len, const float* presence,
                       const float* repetition, dsv_stream_t stream);

/* Every row of out [rows, vocab] becomes the one-point distribution [0, -inf, -inf, ...].   */
int dsv_logits_padding(void* out, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                       dsv_stream_t stream);

/* Compact window index: out[qo[b] + d] = b*T + d for d < qo[b+1] - qo[b] (qo int32/int64,   */
/* [bs + 1]); out holds `total` entries (qo[bs]); writes outside it are dropped.              */
int dsv_window_index(const void* qo_indptr, int32_t qo_i64, int32_t bs, int32_t T, int64_t* out, int64_t total,
                     dsv_stream_t stream);

/* Dense target distribution P [rows, vocab] float32 (out row stride out_stride): softmax of  */
/* the temperature-scaled logits, the backend filter, renormalised (normalize = 0: the       */
/* filtered p as is); greedy rows one-hot at the argmax; unfiltered batches unnormalised.    */
/* Uses the fields of dsv_verify_args up to the history and the workspace; candidates, q,    */
/* uniforms and outputs are ignored.                                                          */
int dsv_target_probs(const dsv_verify_args* args, float* out, int64_t out_stride, int32_t normalize,
                     dsv_stream_t stream);

/* The backend filter on given probabilities probs [rows, vocab] float32 (row stride           */
/* probs_stride; runtime/worker.py:473-508 filter_target_probs), rows = bs * T, the sampling   */
/* parameters per request as in dsv_verify_args (temperatures and the history are ignored:   */
/* each row is filtered at temperature 1, none is greedy).  out [rows, vocab]: the kept      */
/* entries renormalised (normalize = 0: the input values themselves), zeros elsewhere.        */
/* top_p_over_mass = 1 compares the raw mass ranked ahead of an entry with top_p (the         */
/* pytorch backend, flashinfer's joint branch): each row's top_p is divided by its float64    */
/* mass.  Requires a filter flag and rows <= 65535; the workspace holds                       */
/* dsv_filter_workspace_bytes(rows, vocab) bytes.  Entries that round to the same log p tie   */
/* (broken by the lower id).                                                                  */
int64_t dsv_filter_workspace_bytes(int64_t rows, int64_t vocab);
int dsv_filter_probs(const dsv_verify_args* args, const float* probs, int64_t probs_stride, float* out,
                     int64_t out_stride, int32_t normalize, int32_t top_p_over_mass, dsv_stream_t stream);

/* Per row, the ids with p > 0 in id order up to `capacity` ([rows, capacity] int32 ids /   */
/* float32 values, unused slots -1 / 0), lengths = min(n, capacity), overflow = n > capacity  */
/* or any negative / NaN / infinite p.                                                        */
int dsv_compress(const float* p, int64_t rows, int64_t vocab, int64_t row_stride, int32_t capacity, int32_t* ids,
                 float* values, int32_t* lengths, int32_t* overflow, dsv_stream_t stream);

/* Sparse joint target (sampling/sparse/target.py:22-66, CPU form :156-178): from each row's  */
/* top-W of P (top_vals [rows, W] float32 descending, top_ids [rows, W] int64; W <= 64 and    */
/* W <= capacity + 1), keep p > 0, p >= p[top_k - 1] and the nucleus (mass of strictly larger */
/* p < top_p, or top_p >= 1); ids ascending with p / sum(kept) into [rows, capacity] (then    */
/* -1 / 0), lengths = min(count, capacity), overflow = count > capacity.  When P is given,    */
/* overflow rows of P [rows, vocab] become p * (p >= p[top_k - 1]) / sum in place.           */
int dsv_pack_joint(const float* top_vals, const int64_t* top_ids, int64_t rows, int32_t W, const int32_t* top_ks,
                   const float* top_ps, int32_t capacity, int32_t* ids, float* values, int32_t* lengths,
                   int32_t* overflow, float* P, int64_t vocab, int64_t p_stride, dsv_stream_t stream);

/* Chain rejection on given distributions.  P row of draft step s of request b: row_offsets  */
/* [b] + s, else b*T + s.  Packed P (p_ids != NULL) is used on rows whose overflow flag is 0  */
/* (capacity <= 64); other rows read dense_p (divided by denominator[row] when given).  q is  */
/* dense [bs, T-1, vocab] (dense_q) or sparse lanes [bs, T-1, K] (q_ids / q_values).          */
typedef struct dsv_chain_args {
  int32_t bs, T, K, pad0;
  int64_t vocab;
  const int64_t* candidates;  /* [bs, T] */
  const int32_t* verify_lens; /* [bs] in [1, T], NULL = T */
  const float* uniforms;      /* [bs, T-1] */
  const float* uniform_final; /* [bs] */
  const int32_t* prefix_lens; /* [bs] */
  const void* row_offsets;    /* [bs] int32 / int64, NULL = b*T */
  int32_t row_offsets_i64, pad1;
  const float* dense_p;       /* [rows, vocab] (row stride p_stride), or NULL */
  int64_t p_stride;
  const float* denominator;   /* [rows] or NULL */
  const int32_t* p_ids;       /* packed [rows, p_cap], or NULL */
  const float* p_values;
  const int32_t* p_lengths;
  const int32_t* p_overflow;  /* [rows] or NULL (no overflow) */
  int32_t p_cap, pad2;
  const float* dense_q;       /* [bs, T-1, vocab] (row stride q_stride), or NULL */
  int64_t q_stride;
  const void* q_ids;          /* [bs, T-1, K] int32 / int64 */
  int32_t q_ids_i64, pad3;
  const float* q_values;      /* [bs, T-1, K] */
  int32_t* accept;            /* [bs] */
  int32_t* commit;            /* [bs] */
  int64_t* bonus;             /* [bs] */
  int64_t* output;            /* [bs, T] */
  int32_t* new_seq;           /* [bs] */
  /* [bs] or NULL: 1 where the request read a packed row flagged overflow with no dense P to  */
  /* fall back on (the reference stops on the device there, sampling/sparse/accept.py:257,   */
  /* :291; the outputs then come from the row's packed prefix), else 0                       */
  int32_t* overflow_read;
} dsv_chain_args;
int dsv_accept_chain(const dsv_chain_args* args, dsv_stream_t stream);

/* Draft-side K-lane chain over n = bs*(block_size-1) rows of table [n, K, K] (K <= 64):      */
/* out_tok [n] int64, out_q [n, K] float32, confidence [n] float32 (may be NULL).            */
int dsv_sample_chain(const float* table, int64_t n, int32_t K, int32_t block_size, const float* inv_temp,
                     const int32_t* top_k, const float* top_p, const float* min_p, const int32_t* greedy,
                     const float* u, const int64_t* cand, const int64_t* greedy_tok, int64_t* out_tok,
                     float* out_q, float* confidence, dsv_stream_t stream);

/* Factorized draft q table (sampling/factorized/kernels.py:179-300 factor_table, with the     */
/* cancellation fallback of sampling/factorized/cancellation.py:82-147), float64:              */
/* out[n, j, c] = (base[n, c] + a m.TG[c]) / sqrt(d / H + eps), d = first + 2a (xW).m +        */
/* a^2 m.Gram.m, and the direct form head[c].(y / sqrt(mean(y^2) + eps) * norm), y = x + a W m, */
/* where d cancels (d < 2^-24 (|first| + |2a cross| + |a^2 quad|) or not finite).  The cache   */
/* (sampling/factorized/weights.py:34-80 build_cache) holds W [H, R], Gram = W^T W [R, R],      */
/* G, V, TG [vocab, R], bias [R] and norm [H] in float64; head [vocab, H] (bf16 / float32) or  */
/* candidate_head [n K, H].  The workspace arrays are the reference's Workspace fields;        */
/* gemm_ws holds dsv_factor_workspace_doubles(n, K, H, R) doubles.                              */
typedef struct dsv_factor_args {
  int64_t n;                   /* block rows, bs * (T - 1) */
  int32_t K, T, H, R;
  int64_t vocab;
  const void* raw;             /* [bs * T, H] (row stride raw_stride) */
  int32_t raw_dtype, query_dtype;
  int64_t raw_stride;
  const float* rms;            /* [bs * T] */
  const void* query;           /* [bs * T, R] (row stride query_stride) */
  int64_t query_stride;
  const int64_t* anchors;      /* [bs] */
  const int64_t* cand;         /* [n, K] */
  const double* W;             /* cache */
  const double* gram;
  const double* G;
  const double* Vm;
  const double* TG;
  const double* bias;
  const double* norm;
  const void* head;            /* [vocab, H] (row stride head_stride) or NULL with candidate_head */
  const void* candidate_head;  /* [n * K, H] or NULL */
  int32_t head_dtype, pad0;
  int64_t head_stride;
  double eps;
  float* out;                  /* [n, K, K] */
  double* base_out;            /* [n, K] */
  double* x;                   /* [n, H] */
  double* scale;               /* [n] */
  double* first;               /* [n] */
  double* message;             /* [n, K, R] */
  double* tg;                  /* [n, K, R] */
  uint8_t* safe;               /* [n, K] */
  double* d;                   /* [n, K] */
  double* magnitude;           /* [n, K] */
  double* y;                   /* [n, K, H] (the direct form's rows) */
  double* gemm_ws;
  int64_t gemm_ws_doubles;
} dsv_factor_args;
int64_t dsv_factor_workspace_doubles(int64_t n, int32_t K, int32_t H, int32_t R);
int dsv_factor_table(const dsv_factor_args* args, dsv_stream_t stream);
/* The direct form alone (sampling/factorized/cancellation.py:82-147, apply_direct_fallback): */
/* for each (n, j) with safe[n, j] == 0, from x, scale, message and W / norm / head.           */
int dsv_factor_direct(const dsv_factor_args* args, dsv_stream_t stream);
/* The cache's building blocks (weights.py:34-80): out[r, c] = scale * src[r, c] (* mul[c] when */
/* mul is given) widened to float64 (src bf16 / float32, row stride `stride`), and             */
/* C[M, N] (+)= A . B in float64 on the matrix cores, A(m, k) = A[m am + k ak],               */
/* B(k, n) = B[k bk + n bn], C row-major (accumulate != 0: added to C).                         */
int dsv_factor_widen(const void* src, int32_t dtype, int64_t stride, int64_t rows, int64_t cols, double scale,
                     const double* mul, double* out, dsv_stream_t stream);
int dsv_factor_gemm(const double* A, int64_t am, int64_t ak, const double* B, int64_t bk, int64_t bn, double* C,
                    int64_t M, int64_t N, int64_t K, int32_t accumulate, dsv_stream_t stream);

/* SPS verify-length plan (verification/sps.py:35-99: allocate_verify_lens, the calibration   */
/* table lookup it does, the ragged layout's row pointer and _indices), one launch.           */
/* raw [bs, gamma] float32 confidences (row stride raw_stride), probabilities [prob_rows,     */
/* n_bins] float32 (row stride prob_stride), depth [gamma] int64 (rows of the table), optional */
/* boundaries [n_boundaries <= n_bins - 1] float64 ascending (torch.bucketize; NULL: bin =    */
/* trunc(raw * n_bins) clamped).  Survival = running minimum of the running product (float64, */
/* each prefix rounded to float32) of table[depth[d], bin]; the budget - bs positions of      */
/* highest survival (position-major order d * bs + b on ties) are verified beyond each        */
/* request's root: verify_lens [bs] int32 (1 + selected positions), qo_indptr [bs + 1] int32  */
/* (exclusive prefix, may be NULL), window_index [budget] int64 (b * (gamma + 1) + d, may be  */
/* NULL).  bs <= budget <= bs * (gamma + 1).  raw == NULL: verify_lens is an input and only   */
/* the layout (qo_indptr, window_index) is written; window_index holds budget entries, and    */
/* lengths summing past it write only those (qo_indptr[bs] is their sum).                    */
/* bs * gamma + bs <= 38912.                                                                  */
int dsv_sps_plan(const float* raw, int64_t raw_stride, int32_t bs, int32_t gamma, const float* probabilities,
                 int64_t prob_stride, int32_t n_bins, int64_t prob_rows, const int64_t* depth,
                 const double* boundaries, int32_t n_boundaries, int32_t budget, int32_t* verify_lens,
                 int32_t* qo_indptr, int64_t* window_index, dsv_stream_t stream);

/* Draft-side sampling table of the serial last-write refinement (kernels/dspine.py:505-613,  */
/* serial_rs_table), float32 on the matrix cores: out [n, K, K] with n = bs * (T - 1) block    */
/* rows, out[n, j, c] = normalize(raw[r] + rms[r] * ((sigmoid(query[r] + e_j pg^T + gb) *     */
/* (e_j pv^T + res_j res_proj^T)) write_w^T)) * norm_w . head[n, c], r = the row's state row,  */
/* e_j = sqrt(C) * codebook[sender j] (the anchor on a request's first block row, else        */
/* candidate j of the previous row).  raw [bs*T, H], query [bs*T, >= R], codebook [V, C], head */
/* (lm_head [V, H] gathered by cand, or the candidate head [n, K, H] when head_is_candidates)  */
/* and res_emb [V, RR] are bfloat16; the weights float32.  K <= 64; C, H, RR multiples of 16; */
/* R a multiple of 64 up to 512.  workspace: dsv_rs_table_workspace_bytes(n, K, H, R).        */
int64_t dsv_rs_table_workspace_bytes(int64_t n, int32_t K, int32_t H, int32_t R);
int dsv_rs_table(const void* raw, int64_t raw_stride, const float* rms, const void* query, int64_t query_stride,
                 const int64_t* anchors, const int64_t* cand, int64_t n, int32_t K, int32_t T, const void* codebook,
                 int32_t C, const float* pred_gate_w, const float* prev_w, const float* gate_b,
                 const float* write_w, int32_t H, int32_t R, const float* norm_w, const void* head,
                 int32_t head_is_candidates, const void* res_emb, const float* res_proj, int32_t RR, float eps,
                 float* out, void* workspace, int64_t workspace_bytes, dsv_stream_t stream);

/* Commit of an accepted round (SGLang's _commit_accept after the accept / bonus buffers,      */
/* tests/test_tp_accept.py:106-180 of the reference; SGLang is not in the reference, the      */
/* closed form is this build's): request b verified n = verify_lens[b] (NULL: T) positions     */
/* prefix_lens[b] + i with window slots out_cache_loc[slot_offsets[b] + i] (slot_offsets NULL: */
/* b*T + i); the first c = accept[b] + 1 are committed.  out_cache_loc given: req_to_token[    */
/* req_pool_indices[b], prefix + i] = slot for i < c; NULL: the slots are already in the table */
/* and are read from it.  seq_lens[req_pool_indices[b]] = prefix + c (int32 / int64, may be   */
/* NULL); the slots of positions c .. n-1 go to free_slots (int64, in (b, i) order, capacity   */
/* sum(n - c) <= bs*T) and their count to free_count[0] (either may be NULL).                 */
int dsv_commit_accept(int32_t bs, int32_t T, const int32_t* accept, const int32_t* verify_lens,
                      const void* prefix_lens, int32_t prefix_i64, const void* req_pool_indices,
                      int32_t req_pool_i64, int32_t* req_to_token, int64_t rt_stride, int64_t rt_cols,
                      const int64_t* out_cache_loc, const int64_t* slot_offsets, void* seq_lens,
                      int32_t seq_lens_i64, int64_t* free_slots, int32_t* free_count, dsv_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* DSPINE_VERIFY_H */
