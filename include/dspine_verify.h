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
 *   dsv_adjust_logits     sampling/compact.py:14-79 (adjust_logits)
 *   dsv_adjust_history    sampling/compact.py:14-79 with SGLang's presence/repetition buffers
 *                         given as a per-request token history
 *   dsv_target_probs      runtime/worker.py:440-470 (build_dspine_target_probs)
 *   dsv_accept_dense      sampling/rejection.py:101-153 (sample_capped_chain_from_probs)
 *   dsv_accept_sparse     sampling/sparse/accept.py:463-543 (accept_sparse)
 *   dsv_compress          sampling/sparse/accept.py:422-460 (compress_probs)
 *   dsv_sample_chain      kernels/dspine.py:677-772 (serial_sample_chain)
 *   dsv_window_index      verification/sps.py:27-32,87-98 (_indices) and the out_cache_loc
 *                         gather of verification/ragged.py:192-200
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
  /* optional presence / repetition penalty over a token history [bs, hist_len] (-1 = pad) */
  const int32_t* hist_ids;
  int32_t hist_len, pad1;
  const float* presence;         /* [bs]: additive -presence on history tokens */
  const float* repetition;       /* [bs]: x<0 ? x*r : x/r on history tokens */
  /* draft proposal */
  const int64_t* candidates;     /* [bs, T]: anchor then T-1 drafts */
  const void* q_ids;             /* [bs, T-1, K] int32 or int64 */
  int32_t q_ids_i64, K;
  const float* q_values;         /* [bs, T-1, K] */
  const float* uniforms;         /* [bs, T-1] */
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

/* Profiling aid with no counterpart in the reference: the calling thread's later dsv_verify   */
/* calls record `start` / `stop` (hipEvent_t, timing enabled) on their stream right before and */
/* after the chunk-pass kernel, so a benchmark can time that kernel alone.  NULL, NULL: off.   */
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

#ifdef __cplusplus
}
#endif
#endif /* DSPINE_VERIFY_H */
