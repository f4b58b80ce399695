// Commit of an accepted verify round for gfx950: the accepted positions' KV slots into the
// request-to-token table, the new sequence lengths, and the slots of the rejected positions
// compacted into a free list -- what follows the accept / bonus buffers in SGLang's speculative
// worker (its _commit_accept; the accept buffers' layout is pinned by tests/test_tp_accept.py
// :106-180 of the reference).  One workgroup: requests in contiguous ranges a thread, a block
// scan places each request's rejected slots.
#include "dsv_common.h"

namespace dsv {

constexpr int COMMIT_THREADS = 1024;
constexpr int COMMIT_NW = COMMIT_THREADS / WAVE;

__device__ __forceinline__ int64_t load_i(const void* p, int i64, int64_t i) {
  return i64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

__global__ __launch_bounds__(COMMIT_THREADS) void k_commit(int bs, int T, const int32_t* accept,
                                                           const int32_t* verify_lens, const void* prefix_lens,
                                                           int prefix_i64, const void* req_pool, int req_i64,
                                                           int32_t* req_to_token, int64_t rt_stride, int64_t rt_cols,
                                                           const int64_t* out_cache_loc, const int64_t* slot_offsets,
                                                           void* seq_lens, int seq_i64, int64_t* free_slots,
                                                           int32_t* free_count) {
  __shared__ int32_t sred[COMMIT_NW];
  const int tid = threadIdx.x;
  const int per = (bs + COMMIT_THREADS - 1) / COMMIT_THREADS;
  const int b0 = tid * per, b1 = b0 + per < bs ? b0 + per : bs;
  // the request's verified length n and accepted commit c = accept + 1 (clamped into [1, n])
  auto lens_of = [&](int b, int& n, int& c) {
    n = verify_lens ? verify_lens[b] : T;
    n = n < 1 ? 1 : (n > T ? T : n);
    c = accept[b] + 1;
    c = c < 1 ? 1 : (c > n ? n : c);
  };
  int mine = 0;
  for (int b = b0; b < b1; ++b) {
    int n, c;
    lens_of(b, n, c);
    mine += n - c;
  }
  int total = 0;
  int at = block_excl_scan<COMMIT_NW>(mine, sred, &total);
  for (int b = b0; b < b1; ++b) {
    int n, c;
    lens_of(b, n, c);
    const int64_t row = load_i(req_pool, req_i64, b);
    const int64_t pre = load_i(prefix_lens, prefix_i64, b);
    int32_t* rt = req_to_token + row * rt_stride;
    const int64_t base = slot_offsets ? slot_offsets[b] : (int64_t)b * T;  // the request's window slots
    for (int i = 0; i < n; ++i) {
      const int64_t pos = pre + i;
      int64_t slot;
      if (out_cache_loc) {
        slot = out_cache_loc[base + i];
        if (i < c && pos >= 0 && pos < rt_cols) rt[pos] = (int32_t)slot;  // accepted: into the table
      } else {
        slot = (pos >= 0 && pos < rt_cols) ? (int64_t)rt[pos] : -1;  // already in the table
      }
      if (i >= c && free_slots) free_slots[at++] = slot;
    }
    if (seq_lens) {
      const int64_t s = pre + c;
      if (seq_i64)
        reinterpret_cast<int64_t*>(seq_lens)[row] = s;
      else
        reinterpret_cast<int32_t*>(seq_lens)[row] = (int32_t)s;
    }
  }
  if (tid == 0 && free_count) *free_count = total;
}

}  // namespace dsv

using namespace dsv;

extern "C" int dsv_commit_accept(int32_t bs, int32_t T, const int32_t* accept, const int32_t* verify_lens,
                                 const void* prefix_lens, int32_t prefix_i64, const void* req_pool_indices,
                                 int32_t req_pool_i64, int32_t* req_to_token, int64_t rt_stride, int64_t rt_cols,
                                 const int64_t* out_cache_loc, const int64_t* slot_offsets, void* seq_lens,
                                 int32_t seq_lens_i64, int64_t* free_slots, int32_t* free_count,
                                 dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (bs < 0 || T < 1) DSV_FAIL(DSV_ERR_INVALID, "dsv_commit_accept: invalid layout (bs %d, T %d)", bs, T);
  // (bs == 0 still launches: the kernel writes a zero free count, with no memset node that a
  // captured graph would hold)
  if (bs > 0 && (!accept || !prefix_lens || !req_pool_indices || !req_to_token || rt_cols < 1 || rt_stride < rt_cols))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_commit_accept: accept, prefix_lens, req_pool_indices and req_to_token are required");
  hipLaunchKernelGGL(k_commit, dim3(1), dim3(COMMIT_THREADS), 0, stream, bs, T, accept, verify_lens, prefix_lens,
                     prefix_i64, req_pool_indices, req_pool_i64, req_to_token, rt_stride, rt_cols, out_cache_loc,
                     slot_offsets, seq_lens, seq_lens_i64, free_slots, free_count);
  DSV_CHECK_LAUNCH("k_commit");
  return DSV_OK;
}
