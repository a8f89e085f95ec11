// sgemm_skinny.hip -- decode-shaped f32 GEMM (m <= 32) for gfx950.
//
// Replaces the K3 path of MatMul::execute (crates/barracuda/src/ops/
// matmul.rs:65-74 routes m < 256 to shaders/math/matmul_tiled_f64.wgsl,
// where for m <= 32 most of each 16x16 workgroup holds padding rows) for
// small m.  Contract unchanged: C[m,n] = sum_p A[m,p] B[p,n], f32.
//
// The job is streaming B ([k, n], row-major, k*n*4 bytes) from HBM exactly
// once; A (m x k) is tiny and is read through the scalar cache.
//   * A wavefront owns 256 consecutive columns: lane l holds columns
//     4l..4l+3 of every B row it reads (one 1 KB contiguous row segment per
//     wavefront load), with up to 8 row loads in flight per lane.
//   * The four wavefronts of a workgroup take interleaved rows of one
//     k-range (rows k, k+1, k+2, k+3 are read together), then reduce their
//     partial sums through LDS.
//   * The k-range is split over grid.y workgroups so the launch has enough
//     waves to cover 256 CUs; each split writes its m x n partial to the
//     workspace and a second kernel sums the splits in a fixed order, so the
//     result is deterministic.  The split count is bounded so partials stay
//     a few percent of the B stream.
//   * A[i][k] is wave-uniform (k comes from readfirstlane'd wave ids and
//     loop counters), so it is fetched with scalar loads.
#include "bch_internal.h"

#include <stdint.h>

namespace {

constexpr int kCols = 256;  // columns per wavefront (64 lanes x float4)
constexpr int kWaves = 4;
constexpr int kUnroll = 8;

template <int MT>
__global__ __launch_bounds__(256) void sgemm_skinny_partial(
    int M, int N, int K, const float* __restrict__ A, int lda,
    const float* __restrict__ B, int ldb, float* __restrict__ P,
    long long pstride, int kchunk) {
  __shared__ float4 red[kWaves - 1][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = blockIdx.x * kCols + lane * 4;
  const bool nvalid = n < N;
  const int kbeg = blockIdx.y * kchunk;
  const int kend = min(K, kbeg + kchunk);

  float4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);

  for (int k0 = kbeg + wave; k0 < kend; k0 += kWaves * kUnroll) {
    float4 b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int kk = k0 + u * kWaves;
      b[u] = (nvalid && kk < kend)
                 ? bch::load_nt(reinterpret_cast<const float4*>(B + (long long)kk * ldb + n))
                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int kk = k0 + u * kWaves;
      if (kk < kend) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          if (i < M) {
            const float a = A[(long long)i * lda + kk];
            acc[i].x = fmaf(a, b[u].x, acc[i].x);
            acc[i].y = fmaf(a, b[u].y, acc[i].y);
            acc[i].z = fmaf(a, b[u].z, acc[i].z);
            acc[i].w = fmaf(a, b[u].w, acc[i].w);
          }
        }
      }
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i) red[wave - 1][i][lane] = acc[i];
  }
  __syncthreads();
  if (wave == 0 && nvalid) {
    float* p = P + (long long)blockIdx.y * pstride;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (i < M) {
        float4 s = acc[i];
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w) {
          const float4 t = red[w][i][lane];
          s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
        }
        *reinterpret_cast<float4*>(p + (long long)i * N + n) = s;
      }
    }
  }
}

// C[i, n..n+3] = sum over splits s (in order) of P[s][i][n..n+3].
__global__ __launch_bounds__(256) void sgemm_skinny_reduce(
    int M, int N, const float* __restrict__ P, long long pstride, int splits,
    float* __restrict__ C, int ldc) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int n4 = N / 4;
  if (t >= (long long)M * n4) return;
  const int i = (int)(t / n4), n = (int)(t % n4) * 4;
  float4 s = *reinterpret_cast<const float4*>(P + (long long)i * N + n);
  for (int sp = 1; sp < splits; ++sp) {
    const float4 v = *reinterpret_cast<const float4*>(P + sp * pstride + (long long)i * N + n);
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  float* c = C + (long long)i * ldc + n;
  c[0] = s.x; c[1] = s.y; c[2] = s.z; c[3] = s.w;
}

int pick_mt(int m) {
  if (m <= 1) return 1;
  if (m <= 2) return 2;
  if (m <= 4) return 4;
  if (m <= 8) return 8;
  if (m <= 16) return 16;
  return 32;
}

// Split count: enough workgroups to fill the chip (~4 per CU), bounded so
// partial traffic (2 * splits * m * n * 4 bytes) stays <= ~1/16 of B.
int pick_splits(int m, int n, int k) {
  const int colblocks = (n + kCols - 1) / kCols;
  int want = (1024 + colblocks - 1) / colblocks;
  int cap = k / (32 * m);  // 2*s*m*n*4 <= k*n*4/16  <=>  s <= k/(32m)
  int s = want < cap ? want : cap;
  int maxs = k / (kWaves * kUnroll);  // keep >= one unrolled step per wave
  if (s > maxs) s = maxs;
  return s < 1 ? 1 : s;
}

}  // namespace

namespace bch {

size_t sgemm_skinny_workspace_bytes(int m, int n, int k) {
  const int s = pick_splits(m, n, k);
  return sizeof(float) * (size_t)s * (size_t)m * (size_t)n;
}

bool sgemm_skinny_applies(int m, int n, int k, const float* A, int lda,
                          const float* B, int ldb) {
  if (m < 1 || m > 32 || n < 1 || k < 1) return false;
  if (n % 4 != 0 || ldb % 4 != 0) return false;
  if (B && (reinterpret_cast<uintptr_t>(B) & 15) != 0) return false;
  return true;
}

hipError_t launch_sgemm_skinny(hipStream_t s, int m, int n, int k,
                               const float* A, int lda, const float* B,
                               int ldb, float* C, int ldc, void* ws,
                               size_t ws_bytes) {
  const int splits = pick_splits(m, n, k);
  const size_t need = sgemm_skinny_workspace_bytes(m, n, k);
  if (ws == nullptr || ws_bytes < need) return hipErrorInvalidValue;
  float* P = static_cast<float*>(ws);
  const long long pstride = (long long)m * n;
  const int kchunk = (k + splits - 1) / splits;
  dim3 grid((n + kCols - 1) / kCols, splits), block(256);
  switch (pick_mt(m)) {
    case 1: hipLaunchKernelGGL(sgemm_skinny_partial<1>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
    case 2: hipLaunchKernelGGL(sgemm_skinny_partial<2>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
    case 4: hipLaunchKernelGGL(sgemm_skinny_partial<4>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
    case 8: hipLaunchKernelGGL(sgemm_skinny_partial<8>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
    case 16: hipLaunchKernelGGL(sgemm_skinny_partial<16>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
    default: hipLaunchKernelGGL(sgemm_skinny_partial<32>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, pstride, kchunk); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long total = (long long)m * (n / 4);
  hipLaunchKernelGGL(sgemm_skinny_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     m, n, P, pstride, splits, C, ldc);
  return hipGetLastError();
}

}  // namespace bch
