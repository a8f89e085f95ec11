// sdpa_wide.hip -- attention forward for head dimensions above the fused
// kernel's registers (D > 256), in the reference's own three steps on the
// library's MFMA kernels.
//
// The reference's attention ops take any head dimension (ops/attention/
// mod.rs:96-144 checks rank and matching dims only; FlashAttention [S, D],
// ops/flash_attention.rs:57-88; grouped_query_attention/mod.rs:84-147; a
// single-head MultiHeadAttention has D = d_model, ops/mha/mod.rs:152-187).
// The fused kernel (sdpa_fwd.hip) keeps a wavefront's q operand (D/2 floats a
// lane) and its O accumulator (D/2 floats) in registers, which fit up to
// D = 256.  Above that, the scores are materialised one query chunk at a
// time, as the reference's K6 -> K7 -> K9 pipeline does (ops/attention/
// compute.rs:21-111):
//   1. S = Q K^T on the FP32-MFMA GEMM with K as the [n][k] operand (the
//      linear layer's transposed-B tiles), batched over key/value heads;
//   2. S = scale * S with the causal mask (keys past the query set to -inf),
//      then the HBM-streaming row softmax in place -- one pass where the
//      scores' rows take the wavefront-per-row kernel (the scale and mask
//      applied as it loads them), else a scale-and-mask pass first;
//   3. O = P V on the same GEMM, written through O's row stride.
// At D > 256 the two products carry 4 D flops per score against about 16
// bytes of score traffic (stored, normalised in place, read back),
// above the FP32 ridge of 19.7 FLOP/B, so the GEMMs dominate.  Measured at
// B=4, H=32, S=2048, D=512 (one box): 8.81 ms non-causal (79.4% of FP32 MFMA
// peak), 5.71 ms causal (61.3%); 9.76 / 6.21 ms with the scale and mask in a
// pass of their own.
//
// Layout of the passes: for each batch b and query head g of a key/value
// group (query head h = hk * G + g reads key/value head hk), one batched GEMM
// runs over the Hkv key/value heads (A stride G * q.head, B stride k.head),
// on query rows [r0, r1) at a time so the chunk's scores fit kWideScoreCap.
// Causal chunks need only keys [0, r1): their products are cut to n = r1.
#include "bch_internal.h"

#include <algorithm>

namespace {

// Scores of one pass are capped at this many bytes (the query chunk shrinks
// to fit; at least one row).
constexpr size_t kWideScoreCap = (size_t)256 << 20;

// Query rows per pass are also capped so that (key/value heads x rows) stays
// within kWideMaxRows rows of scores.
constexpr long long kWideMaxRows = 1LL << 22;

// x *= scale in place over [rows][n]; with causal, row r (query r0 + r % m)
// masks keys j > r0 + r % m to -inf.  A workgroup of 256 per row, the grid
// striding over the rows.
__global__ __launch_bounds__(256) void sdpa_scale_mask_kernel(float* __restrict__ s, long long rows, int n, int m,
                                                              int r0, float scale, int causal) {
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    float* row = s + r * n;
    const int lim = causal ? r0 + (int)(r % m) : 0x7fffffff;  // last allowed key
    for (int j = threadIdx.x; j < n; j += 256) row[j] = j > lim ? -INFINITY : row[j] * scale;
  }
}

struct WidePlan {
  int rows = 0;          // query rows per chunk
  size_t score_bytes = 0;  // scores of one chunk, 256-byte aligned
  size_t extra_bytes = 0;  // the GEMMs' and the softmax's own scratch
};

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The chunk of query rows [r0, r0 + m) and its keys [0, n).
void chunk_shape(const WidePlan& p, int Sq, int Skv, bool causal, int r0, int& m, int& n) {
  m = std::min(p.rows, Sq - r0);
  n = causal ? std::min(Skv, r0 + m) : Skv;
}

// lda / ldb: the row strides of q and k (the [n][k] operand), which pick the
// GEMM's path for the first product.
WidePlan wide_plan(int Hkv, int Sq, int Skv, int D, bool causal, int lda, int ldb) {
  WidePlan p;
  const size_t per_row = (size_t)Hkv * Skv * sizeof(float);
  long long rows = (long long)std::max<size_t>(1, kWideScoreCap / per_row);
  rows = std::min(rows, std::max(1LL, kWideMaxRows / Hkv));
  // causal chunks are cut to their keys; smaller chunks waste less of the square
  if (causal) rows = std::min<long long>(rows, std::max(256, (Sq / 4 + 255) / 256 * 256));
  if (rows >= 256) rows = rows / 256 * 256;
  p.rows = (int)std::min<long long>(rows, Sq);
  p.score_bytes = align256((size_t)Hkv * p.rows * Skv * sizeof(float));
  // the scratch of the three steps, at every chunk the launch will run (a
  // short last chunk can take the skinny GEMMs, whose partials need more);
  // pointers are taken as aligned, which admits every kernel path a launch
  // can take
  size_t x = 0;
  for (int r0 = 0; r0 < Sq; r0 += p.rows) {
    int m, n;
    chunk_shape(p, Sq, Skv, causal, r0, m, n);
    x = std::max(x, bch::sgemm_ex_workspace_bytes(true, Hkv, m, n, D, lda, ldb));
    x = std::max(x, bch::sgemm_workspace_bytes(Hkv, m, D, n));
    x = std::max(x, bch::softmax_workspace_bytes((long long)Hkv * m, n));
  }
  p.extra_bytes = x;
  return p;
}

}  // namespace

namespace bch {

size_t sdpa_wide_workspace_bytes(int Hkv, int Sq, int Skv, int D, int causal, long long q_row, long long k_row) {
  if (q_row > 0x7fffffffLL || k_row > 0x7fffffffLL) return 0;
  const WidePlan p = wide_plan(Hkv, Sq, Skv, D, causal != 0, (int)q_row, (int)k_row);
  return p.score_bytes + p.extra_bytes;
}

hipError_t launch_sdpa_wide(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                            const float* q, const float* k, const float* v, float* o, const SdpaStrides& st,
                            void* ws, size_t ws_bytes) {
  if (Hkv < 1 || H % Hkv != 0 || Hkv > 65535) return hipErrorInvalidValue;
  if (st.q.row > 0x7fffffffLL || st.k.row > 0x7fffffffLL || st.v.row > 0x7fffffffLL || st.o.row > 0x7fffffffLL)
    return hipErrorInvalidValue;
  const int G = H / Hkv;
  const int qr = (int)st.q.row, kr = (int)st.k.row, vr = (int)st.v.row, orow = (int)st.o.row;
  const WidePlan p = wide_plan(Hkv, Sq, Skv, D, causal != 0, qr, kr);
  if (ws == nullptr || ws_bytes < p.score_bytes + p.extra_bytes) return hipErrorInvalidValue;
  float* S = static_cast<float*>(ws);
  void* xws = static_cast<char*>(ws) + p.score_bytes;
  const size_t xbytes = ws_bytes - p.score_bytes;
  for (int b = 0; b < B; ++b) {
    for (int g = 0; g < G; ++g) {
      // query head hk * G + g of batch b, for hk < Hkv (batched)
      const float* qb = q + b * st.q.batch + (long long)g * st.q.head;
      float* ob = o + b * st.o.batch + (long long)g * st.o.head;
      const float* kb = k + b * st.k.batch;
      const float* vb = v + b * st.v.batch;
      for (int r0 = 0; r0 < Sq; r0 += p.rows) {
        int m, n;
        chunk_shape(p, Sq, Skv, causal != 0, r0, m, n);
        const long long per = (long long)m * n;
        hipError_t e = launch_sgemm_ex(s, true, Hkv, m, n, D, qb + (long long)r0 * qr, qr, G * st.q.head, kb, kr,
                                       st.k.head, nullptr, kActNone, S, n, per, xws, xbytes);
        if (e != hipSuccess) return e;
        const long long rows = (long long)Hkv * m;
        if (softmax_rows_scaled_supported(n, S, S)) {
          // scale and mask on the softmax's own load: one pass over the scores
          e = launch_softmax_rows_scaled(s, rows, n, S, S, scale, causal, m, r0);
        } else {
          hipLaunchKernelGGL(sdpa_scale_mask_kernel, dim3((unsigned)std::min(rows, 65536LL)), dim3(256), 0, s, S,
                             rows, n, m, r0, scale, causal);
          e = hipGetLastError();
          if (e != hipSuccess) return e;
          e = launch_softmax_rows(s, rows, n, S, S, xws, xbytes);
        }
        if (e != hipSuccess) return e;
        e = launch_sgemm(s, Hkv, m, D, n, S, n, per, vb, vr, st.v.head, ob + (long long)r0 * orow, orow,
                         G * st.o.head, xws, xbytes);
        if (e != hipSuccess) return e;
      }
    }
  }
  return hipSuccess;
}

}  // namespace bch
