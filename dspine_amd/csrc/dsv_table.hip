// Draft-side sampling table of the serial last-write refinement for gfx950
// (kernels/dspine.py:505-613, serial_rs_table): for every block row n and sender lane j,
//   e      = sqrt(C) * codebook[sender]                            [C]
//   gate   = sigmoid(q[n] + e @ pg^T + gb),  value = e @ pv^T (+ res_emb[sender] @ res_proj^T)
//   msg    = gate * value                                          [R]
//   ref    = x[n] + scale[n] * (msg @ w_last^T)                    [H]
//   T[n, j, c] = (ref / sqrt(mean(ref^2) + eps) * norm_w) . head[n, c]
// in float32 on the matrix cores (v_mfma_f32_16x16x4f32), three launches:
//   k_rs_message  sender rows x R: the gathered, scaled codebook rows times [pg; pv]^T (the pg / pv
//                 rows staged in LDS tiles shared by a workgroup's waves), with the gate, the value
//                 and their product in the epilogue -> msg [n*K, R]
//   k_rs_table    (row, 16 senders, H slice): msg times w_last^T (w_last staged in LDS tiles of 16
//                 rows shared by a workgroup's four units) in 16 x 16 output blocks that are
//                 already the B operand of the second product against the 16 candidates' head
//                 rows, so ref never leaves registers; partial sums of ref^2 and of the dot products
//   k_rs_finish   the slices combined, divided by sqrt(mean + eps)
//
// MFMA operand layout (16x16x4, one wave): lane l holds A[l % 16][k] and B[k][l % 16] for k of its
// lane group g = l / 16, and receives D[4g + v][l % 16], v = 0..3.  A product of 16 k values is
// four instructions; lane group g takes k = 4g + s at step s (a permutation of k that A and B
// share), so every lane loads its 4 k values as one contiguous vector.
#include <math.h>
#include <string.h>

#include "dsv_common.h"

namespace dsv {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int RS_RMAX = 512;  // R held in registers by k_rs_table (R / 4 floats a lane)

struct RsArgs {
  const uint16_t* raw;   // [m, H] bf16 bits (row stride raw_stride)
  const float* rms;      // [m]
  const uint16_t* query; // [m, >= R] bf16 bits (row stride query_stride)
  const int64_t* anchors;  // [bs]
  const int64_t* cand;     // [n, K]
  const uint16_t* codebook;  // [V, C] bf16 bits
  const float* pg;         // [R, C]
  const float* pv;         // [R, C]
  const float* gb;         // [R]
  const float* w_last;     // [H, R]
  const float* norm_w;     // [H]
  const uint16_t* head;    // lm_head [V, H] bf16 bits, or the candidate head [n, K, H]
  const uint16_t* res_emb; // [V, RR] bf16 bits or NULL
  const float* res_proj;   // [R, RR]
  int64_t raw_stride, query_stride;
  int32_t T, K, H, R, C, RR;
  int32_t n, head_is_cand;
  float eps, sqrt_c;
  float* msg;       // [n * K, R] workspace
  float* part;      // [slices, units, 16 + 16 * KB * 16] workspace
  float* out;       // [n, K, K]
  int32_t KB;       // ceil(K / 16): candidate blocks
  int32_t units;    // n * KB: (row, 16-sender block) pairs
  int32_t slices, hs;  // H slices of hs columns
};

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ f4 bf4(const uint16_t* p) {  // 4 bf16 (8-byte aligned)
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  return f4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u), __uint_as_float(w.y << 16),
            __uint_as_float(w.y & 0xFFFF0000u)};
}
__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 mfma4(f4 a, f4 b, f4 c) {
  // the four k steps of a 16-wide k chunk
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
}

// The sender token of sender row i = n * K + j: the anchor on a request's first block row, else
// candidate j of the previous row.
__device__ __forceinline__ int64_t sender_of(const RsArgs& A, int64_t i) {
  const int64_t n = i / A.K, j = i - n * A.K;
  const int tm = (int)(n % (A.T - 1));
  return tm == 0 ? A.anchors[n / (A.T - 1)] : A.cand[(n - 1) * A.K + j];
}
// The state row (of the [bs*T] rows) block row n refines.
__device__ __forceinline__ int64_t state_row(const RsArgs& A, int64_t n) {
  return n / (A.T - 1) * A.T + 1 + n % (A.T - 1);
}

// ---------------------------------------------------------------------------------------
// k_rs_message: 64 sender rows x 64 R columns a workgroup (wave w: sender rows 16w..16w+15).
// The B operands (pg and pv rows r0..r0+63) go through LDS in tiles of 64 k, shared by the four
// waves, the next tile's loads in flight in registers while the current one is used.
// ---------------------------------------------------------------------------------------
constexpr int RS_MK = 64;            // k of a staged tile (four 16-wide k steps)
constexpr int RS_MROW = RS_MK + 4;   // LDS row stride (floats): a lane group's 16 rows of one
                                     // k step fall in distinct bank groups
constexpr int RS_MCH = 2 * 64 * RS_MK / 4 / 256;  // 16-byte chunks of a tile pair a thread copies

__global__ __launch_bounds__(256) void k_rs_message(RsArgs A) {
  __shared__ __align__(16) float bt[2 * 64 * RS_MROW];  // pg tile, then pv tile
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const int64_t Ns = (int64_t)A.n * A.K;
  const int64_t i = (int64_t)blockIdx.x * 64 + w * 16 + li;  // the A-operand row of this lane
  const bool live = i < Ns;
  const int64_t sid = live ? sender_of(A, i) : 0;
  const int r0 = blockIdx.y * 64;
  const uint16_t* erow = A.codebook + sid * A.C;
  f4 accg[4], accv[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) accg[cb] = accv[cb] = f4{0.f, 0.f, 0.f, 0.f};
  // tile copy: chunk q = c * 256 + tid -> matrix q / 1024, row (q % 1024) / 16, k chunk q % 16
  f4 pre[RS_MCH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int c = 0; c < RS_MCH; ++c) {
      const int q = c * 256 + tid, mat = q >> 10, row = (q >> 4) & 63, kc = q & 15;
      const float* src = mat ? A.pv : A.pg;
      if (k0 + 4 * kc < A.C) pre[c] = ld4(src + (int64_t)(r0 + row) * A.C + k0 + 4 * kc);
    }
  };
  fetch(0);
  for (int k0 = 0; k0 < A.C; k0 += RS_MK) {
    __syncthreads();  // (the previous tile's readers are done)
#pragma unroll
    for (int c = 0; c < RS_MCH; ++c) {
      const int q = c * 256 + tid, mat = q >> 10, row = (q >> 4) & 63, kc = q & 15;
      if (k0 + 4 * kc < A.C) *reinterpret_cast<f4*>(bt + (mat * 64 + row) * RS_MROW + 4 * kc) = pre[c];
    }
    __syncthreads();
    if (k0 + RS_MK < A.C) fetch(k0 + RS_MK);  // in flight under this tile's products
    const int ns = (A.C - k0) / 16 < RS_MK / 16 ? (A.C - k0) / 16 : RS_MK / 16;
#pragma unroll 1
    for (int st = 0; st < ns; ++st) {  // (ns < 4: a partial last tile when C is not a multiple of RS_MK)
      f4 a = bf4(erow + k0 + 16 * st + 4 * g);
      a *= A.sqrt_c;
      if (!live) a = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const float* bp = bt + (16 * cb + li) * RS_MROW + 16 * st + 4 * g;
        accg[cb] = mfma4(a, *reinterpret_cast<const f4*>(bp), accg[cb]);
        accv[cb] = mfma4(a, *reinterpret_cast<const f4*>(bp + 64 * RS_MROW), accv[cb]);
      }
    }
  }
  if (A.res_emb) {  // the terminal residual: value += res_emb[sender] @ res_proj^T
    const uint16_t* rrow = A.res_emb + sid * A.RR;
    for (int k0 = 0; k0 < A.RR; k0 += 16) {
      f4 a = bf4(rrow + k0 + 4 * g);
      if (!live) a = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int64_t r = r0 + 16 * cb + li;
        accv[cb] = mfma4(a, ld4(A.res_proj + r * A.RR + k0 + 4 * g), accv[cb]);
      }
    }
  }
  // lane: D[4g + v][li] = sender row 16w + 4g + v, column r0 + 16cb + li
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t io = (int64_t)blockIdx.x * 64 + w * 16 + 4 * g + v;
    if (io >= Ns) continue;
    const int64_t mrow = state_row(A, io / A.K);
    const uint16_t* qrow = A.query + mrow * A.query_stride;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int r = r0 + 16 * cb + li;
      const float pre_ = (bf(qrow[r]) + accg[cb][v]) + A.gb[r];
      const float gate = 1.f / (1.f + expf(-pre_));
      A.msg[io * A.R + r] = gate * accv[cb][v];
    }
  }
}

// ---------------------------------------------------------------------------------------
// k_rs_table: one (row, 16-sender block) a wave, 4 a workgroup, one H slice a grid column.  The
// workgroup stages each 16-row tile of w_last (16 h x R) in LDS once for its four waves, the
// next tile's loads in flight in registers while the current tile feeds the matrix cores.
// ---------------------------------------------------------------------------------------
constexpr int RS_TROW = RS_RMAX + 4;  // LDS row stride of a w_last tile (floats): 16 rows' 16-byte
                                      // A fragments of one k step fall in distinct bank groups
constexpr int RS_TCH = 16 * RS_RMAX / 4 / 256;  // 16-byte chunks of a full tile a thread copies

template <int KB>
__global__ __launch_bounds__(256) void k_rs_table(RsArgs A) {
  __shared__ __align__(16) float tile[16 * RS_TROW];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const int unit = blockIdx.x * 4 + w;
  const bool ulive = unit < A.units;  // (a wave past the last unit still copies tiles)
  const int slice = blockIdx.y;
  const int64_t n = ulive ? unit / KB : 0;
  const int jb = ulive ? unit - (int)n * KB : 0;
  const int j = jb * 16 + li;  // the sender lane of this lane's B-operand column
  const bool jlive = ulive && j < A.K;
  const int64_t mrow = state_row(A, n);
  const float scale = A.rms[mrow];
  const uint16_t* xrow = A.raw + mrow * A.raw_stride;
  // msg of sender j in registers: lane group g holds columns 16t + 4g .. 16t + 4g + 3
  f4 mb[RS_RMAX / 16];
  const float* mrowp = A.msg + (n * A.K + (jlive ? j : 0)) * A.R;
#pragma unroll
  for (int t = 0; t < RS_RMAX / 16; ++t) {
    mb[t] = f4{0.f, 0.f, 0.f, 0.f};
    if (16 * t < A.R && jlive) mb[t] = ld4(mrowp + 16 * t + 4 * g);
  }
  // the candidates' head rows (A operand of the second product: row c = cb*16 + li)
  const uint16_t* hrow[KB];
  bool clive[KB];
#pragma unroll
  for (int cb = 0; cb < KB; ++cb) {
    const int c = cb * 16 + li;
    clive[cb] = ulive && c < A.K;
    const int64_t cc = clive[cb] ? c : 0;
    hrow[cb] = A.head_is_cand ? A.head + (n * A.K + cc) * A.H : A.head + A.cand[n * A.K + cc] * A.H;
  }
  f4 dot[KB];
#pragma unroll
  for (int cb = 0; cb < KB; ++cb) dot[cb] = f4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;
  const int h_lo = slice * A.hs, h_hi = h_lo + A.hs;
  // tile copy: chunk q = i * 256 + tid of the tile's 16 x R/4 chunks -> row q / (R/4), column
  // chunk q % (R/4); chunks past 4R (R < RS_RMAX) are not copied (goff -1)
  const int rq = A.R / 4, nq = 16 * rq;
  int goff[RS_TCH], loff[RS_TCH];  // this thread's chunks: offsets in w_last rows h0.. and in the tile
#pragma unroll
  for (int i = 0; i < RS_TCH; ++i) {
    const int q = i * 256 + tid;
    const int row = q / rq, col = q - row * rq;
    goff[i] = q < nq ? row * A.R + 4 * col : -1;
    loff[i] = row * RS_TROW + 4 * col;
  }
  f4 pre[RS_TCH];
  auto fetch = [&](int h0) {
    const float* base = A.w_last + (int64_t)h0 * A.R;
#pragma unroll
    for (int i = 0; i < RS_TCH; ++i)
      if (goff[i] >= 0) pre[i] = ld4(base + goff[i]);
  };
  fetch(h_lo);
  for (int h0 = h_lo; h0 < h_hi; h0 += 16) {
    __syncthreads();  // (the previous tile's readers are done)
#pragma unroll
    for (int i = 0; i < RS_TCH; ++i)
      if (goff[i] >= 0) *reinterpret_cast<f4*>(tile + loff[i]) = pre[i];
    __syncthreads();
    if (h0 + 16 < h_hi) fetch(h0 + 16);  // in flight under this tile's products
    if (!ulive) continue;
    // ref^T block [16 h x 16 senders]: A = w_last rows h0 + li (from the tile), B = msg^T
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    const float* arow = tile + li * RS_TROW + 4 * g;
#pragma unroll
    for (int t = 0; t < RS_RMAX / 16; ++t)
      if (16 * t < A.R) acc = mfma4(*reinterpret_cast<const f4*>(arow + 16 * t), mb[t], acc);
    // lane: h = h0 + 4g + v, sender j; ref, its square, and ref * norm_w as the B operand
    const f4 xv = bf4(xrow + h0 + 4 * g);
    const f4 nw = ld4(A.norm_w + h0 + 4 * g);
    f4 bv;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float ref = xv[v] + scale * acc[v];
      ss += ref * ref;
      bv[v] = ref * nw[v];
    }
#pragma unroll
    for (int cb = 0; cb < KB; ++cb) {
      f4 a = bf4(hrow[cb] + h0 + 4 * g);
      if (!clive[cb]) a = f4{0.f, 0.f, 0.f, 0.f};
      dot[cb] = mfma4(a, bv, dot[cb]);
    }
  }
  if (!ulive) return;
  // the slice's partial sums: ss over the lane group's h (lanes li, li+16, li+32, li+48 share j),
  // dot[cb][v] = sum_h head[c = cb*16 + 4g + v][h] * ref[j][h] * norm_w[h]
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  float* pp = A.part + ((int64_t)slice * A.units + unit) * (16 + 16 * KB * 16);
  if (g == 0) pp[li] = ss;
#pragma unroll
  for (int cb = 0; cb < KB; ++cb)
#pragma unroll
    for (int v = 0; v < 4; ++v) pp[16 + (cb * 16 + 4 * g + v) * 16 + li] = dot[cb][v];
}

// out[n, j, c] = (sum over slices of the dot products) / sqrt(sum of ref^2 / H + eps)
__global__ void k_rs_finish(RsArgs A) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // n * K * K + j * K + c
  const int64_t total = (int64_t)A.n * A.K * A.K;
  if (e >= total) return;
  const int64_t n = e / ((int64_t)A.K * A.K);
  const int j = (int)(e / A.K % A.K), c = (int)(e % A.K);
  const int unit = (int)n * A.KB + j / 16, jl = j % 16;
  const int stride = 16 + 16 * A.KB * 16;
  float ss = 0.f, d = 0.f;
  for (int s = 0; s < A.slices; ++s) {
    const float* pp = A.part + ((int64_t)s * A.units + unit) * stride;
    ss += pp[jl];
    d += pp[16 + c * 16 + jl];
  }
  A.out[e] = d / sqrtf(ss / (float)A.H + A.eps);
}

}  // namespace dsv

using namespace dsv;

extern "C" int64_t dsv_rs_table_workspace_bytes(int64_t n, int32_t K, int32_t H, int32_t R) {
  const int64_t KB = (K + 15) / 16;
  const int64_t slices = H % 128 == 0 ? 8 : 1;
  return n * K * R * 4 + slices * n * KB * (16 + 16 * KB * 16) * 4 + 256;
}

extern "C" int dsv_rs_table(const void* raw, int64_t raw_stride, const float* rms, const void* query,
                            int64_t query_stride, const int64_t* anchors, const int64_t* cand, int64_t n, int32_t K,
                            int32_t T, const void* codebook, int32_t C, const float* pred_gate_w, const float* prev_w,
                            const float* gate_b, const float* write_w, int32_t H, int32_t R, const float* norm_w,
                            const void* head, int32_t head_is_candidates, const void* res_emb, const float* res_proj,
                            int32_t RR, float eps, float* out, void* workspace, int64_t workspace_bytes,
                            dsv_stream_t stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (n < 0 || K < 1 || K > 64 || T < 2 || n % (T - 1))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_rs_table: layout mismatch (n %lld, K %d, T %d)", (long long)n, K, T);
  if (n == 0) return DSV_OK;
  if (!raw || !rms || !query || !anchors || !cand || !codebook || !pred_gate_w || !prev_w || !gate_b || !write_w ||
      !norm_w || !head || !out || !workspace || (res_emb && !res_proj))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_rs_table: required pointer is null");
  if (C < 16 || C % 16 || H < 16 || H % 16 || R < 64 || R % 64 || R > RS_RMAX || (res_emb && (RR < 16 || RR % 16)))
    DSV_FAIL(DSV_ERR_UNSUPPORTED,
             "dsv_rs_table: needs C, H (and the residual width) multiples of 16 and R a multiple of 64 up to %d "
             "(C %d, H %d, R %d)", RS_RMAX, C, H, R);
  if (raw_stride < H || query_stride < R || (uintptr_t)raw % 8 || (uintptr_t)query % 8 || (uintptr_t)codebook % 8 ||
      (uintptr_t)head % 8 || raw_stride % 4 || (res_emb && (uintptr_t)res_emb % 8))
    DSV_FAIL(DSV_ERR_INVALID, "dsv_rs_table: bf16 operands need 8-byte aligned rows");
  if (workspace_bytes < dsv_rs_table_workspace_bytes(n, K, H, R))
    DSV_FAIL(DSV_ERR_WORKSPACE, "dsv_rs_table: workspace too small");
  RsArgs A;
  memset(&A, 0, sizeof(A));
  A.raw = reinterpret_cast<const uint16_t*>(raw);
  A.rms = rms;
  A.query = reinterpret_cast<const uint16_t*>(query);
  A.anchors = anchors;
  A.cand = cand;
  A.codebook = reinterpret_cast<const uint16_t*>(codebook);
  A.pg = pred_gate_w;
  A.pv = prev_w;
  A.gb = gate_b;
  A.w_last = write_w;
  A.norm_w = norm_w;
  A.head = reinterpret_cast<const uint16_t*>(head);
  A.res_emb = reinterpret_cast<const uint16_t*>(res_emb);
  A.res_proj = res_proj;
  A.raw_stride = raw_stride;
  A.query_stride = query_stride;
  A.T = T;
  A.K = K;
  A.H = H;
  A.R = R;
  A.C = C;
  A.RR = res_emb ? RR : 0;
  A.n = (int32_t)n;
  A.head_is_cand = head_is_candidates ? 1 : 0;
  A.eps = eps;
  A.sqrt_c = (float)sqrt((double)C);
  A.KB = (K + 15) / 16;
  A.units = (int32_t)n * A.KB;
  A.slices = H % 128 == 0 ? 8 : 1;
  A.hs = H / A.slices;
  char* ws = reinterpret_cast<char*>(workspace);
  A.msg = reinterpret_cast<float*>(ws);
  A.part = reinterpret_cast<float*>(ws + (((int64_t)n * K * R * 4 + 255) / 256) * 256);
  A.out = out;
  const int64_t Ns = n * K;
  hipLaunchKernelGGL(k_rs_message, dim3((unsigned)((Ns + 63) / 64), (unsigned)(R / 64)), dim3(256), 0, stream, A);
  DSV_CHECK_LAUNCH("k_rs_message");
  const dim3 tg((unsigned)((A.units + 3) / 4), (unsigned)A.slices);
  switch (A.KB) {
    case 1: hipLaunchKernelGGL(k_rs_table<1>, tg, dim3(256), 0, stream, A); break;
    case 2: hipLaunchKernelGGL(k_rs_table<2>, tg, dim3(256), 0, stream, A); break;
    case 3: hipLaunchKernelGGL(k_rs_table<3>, tg, dim3(256), 0, stream, A); break;
    default: hipLaunchKernelGGL(k_rs_table<4>, tg, dim3(256), 0, stream, A); break;
  }
  DSV_CHECK_LAUNCH("k_rs_table");
  const int64_t total = n * K * K;
  hipLaunchKernelGGL(k_rs_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, A);
  DSV_CHECK_LAUNCH("k_rs_finish");
  return DSV_OK;
}
