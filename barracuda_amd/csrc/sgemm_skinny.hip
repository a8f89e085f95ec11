// sgemm_skinny.hip -- decode-shaped f32 GEMM (m <= 32) for gfx950.
//
// Replaces the K3 path of MatMul::execute (crates/barracuda/src/ops/
// matmul.rs:65-74 routes m < 256 to shaders/math/matmul_tiled_f64.wgsl,
// where for m <= 32 most of each 16x16 workgroup holds padding rows) for
// small m.  Contract unchanged: C[m,n] = sum_p A[m,p] B[p,n], f32.
//
// The job is streaming B ([k, n] row-major, k*n*4 bytes) from HBM once.
// Two kernels write split-k partials; a third sums them in split order, so
// the result is deterministic:
//   * m <= 4, sgemm_skinny_fma: a wavefront owns 256 columns (lane l holds
//     columns 4l..4l+3, one 1 KB row segment per load); the four wavefronts
//     of a workgroup take interleaved rows with 8 row loads in flight; A[i][k]
//     is wave-uniform and comes through the scalar cache.
//   * 4 < m <= 32, sgemm_skinny_mfma: at 2m multiply-adds per B element the
//     non-packed FP32 VALU cannot keep up with HBM, so v_mfma_f32_16x16x4_f32
//     computes C^T = B^T A^T (m padded to 16 or 32).  Lane l = 16q + i loads
//     float4 B[k][n0 + 4i .. +3] and feeds component c to MFMA block c; in a
//     16-row chunk lane quarter q takes rows 4q + s in step s.  The four
//     wavefronts of a workgroup cover 4 x 64 adjacent columns of the same
//     rows (1 KB per row per workgroup).  The workgroup's A^T slice is staged
//     once in LDS (zero past m and past the k range), so every chunk is
//     branch-free: B rows past the range are clamped to the last valid row
//     (an L2 hit) and meet zeros in A.  B loads run PF chunks ahead.
//   * Measured on MI355X (K 4096, N 11008, weights rotated past the 256 MB
//     Infinity Cache): cross-XCD release/acquire fences for an in-kernel
//     "last workgroup reduces" cost ~75 us per call, so the split reduction
//     is a separate launch (~3 us).
#include "bch_internal.h"

#include <stdint.h>

namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kFmaCols = 256;   // columns per workgroup, FMA kernel
constexpr int kFmaUnroll = 8;
constexpr int kMmaCols = 256;   // columns per workgroup, MFMA kernel (4 x 64)
constexpr int kStageF4 = 16;    // float4 of A staged per thread (MFMA kernel)
constexpr int kPF = 2;          // chunks of B in flight ahead of the MFMAs

// ---------------------------------------------------------------- m <= 4
template <int MT>
__global__ __launch_bounds__(256) void sgemm_skinny_fma(int M, int N, int K, const float* __restrict__ A,
                                                        int lda, const float* __restrict__ B, int ldb,
                                                        float* __restrict__ P, int kchunk) {
  __shared__ float4 red[3][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = blockIdx.x * kFmaCols + lane * 4;
  const bool nvalid = n < N;
  const int kbeg = blockIdx.y * kchunk, kend = min(K, kbeg + kchunk);
  float4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = kbeg + wave; k0 < kend; k0 += 4 * kFmaUnroll) {
    float4 b[kFmaUnroll];
#pragma unroll
    for (int u = 0; u < kFmaUnroll; ++u) {
      const int kk = k0 + 4 * u;
      b[u] = (nvalid && kk < kend) ? bch::load_nt(reinterpret_cast<const float4*>(B + (long long)kk * ldb + n))
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kFmaUnroll; ++u) {
      const int kk = k0 + 4 * u;
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
    float* p = P + (long long)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (i < M) {
        float4 s = acc[i];
#pragma unroll
        for (int w = 0; w < 3; ++w) {
          const float4 t = red[w][i][lane];
          s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
        }
        *reinterpret_cast<float4*>(p + (long long)i * N + n) = s;
      }
    }
  }
}

// ---------------------------------------------------------------- 4 < m <= 32
template <int MB>  // m blocks of 16
__global__ __launch_bounds__(256) void sgemm_skinny_mfma(int M, int N, int K, const float* __restrict__ A,
                                                         int lda, const float* __restrict__ B, int ldb,
                                                         float* __restrict__ P, int kchunk, int avec) {
  extern __shared__ float4 smem4[];
  float* xs = reinterpret_cast<float*>(smem4);  // [16 MB][nch*16 + 4]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane >> 4, li = lane & 15;
  const int n0 = blockIdx.x * kMmaCols + 64 * wave;
  const int nl = min(n0 + 4 * li, N - 4);  // columns past N are computed and dropped
  const int kbeg = blockIdx.y * kchunk, kend = min(K, kbeg + kchunk);
  const int nch = kend > kbeg ? (kend - kbeg + 15) / 16 : 0;
  const int ld = nch * 16 + 4;

  // stage A^T: all loads issued before the LDS writes
  {
    const int q4 = nch * 4;
    const int total = MB * 16 * q4;
    float4 r[kStageF4];
#pragma unroll
    for (int u = 0; u < kStageF4; ++u) {
      const int e = tid + u * 256;
      const int m = q4 ? e / q4 : 0, kq = q4 ? e % q4 : 0;
      const int kk = kbeg + 4 * kq;
      const float* ar = A + (long long)m * lda + kk;
      if (e < total && m < M && kk + 3 < kend && avec) {
        r[u] = *reinterpret_cast<const float4*>(ar);
      } else {
        float t[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) t[q] = (e < total && m < M && kk + q < kend) ? ar[q] : 0.f;
        r[u] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
#pragma unroll
    for (int u = 0; u < kStageF4; ++u) {
      const int e = tid + u * 256;
      if (e < total) *reinterpret_cast<float4*>(xs + (e / q4) * ld + 4 * (e % q4)) = r[u];
    }
  }
  __syncthreads();

  f32x4v acc[4][MB];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[c][b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  if (nch > 0) {
    const int klast = kend - 1;
    const float* Bl = B + nl;
    constexpr int NB = kPF + 1;
    float4 w[NB][4];
    auto load = [&](int slot, int j) {
      const int k16 = kbeg + 16 * j + 4 * lq;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        w[slot][s] = bch::load_nt(reinterpret_cast<const float4*>(Bl + (long long)min(k16 + s, klast) * ldb));
    };
    auto mma = [&](int slot, int j) {
      float4 x[MB];
#pragma unroll
      for (int b = 0; b < MB; ++b) x[b] = *reinterpret_cast<const float4*>(xs + (16 * b + li) * ld + 16 * j + 4 * lq);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float ws[4] = {w[slot][s].x, w[slot][s].y, w[slot][s].z, w[slot][s].w};
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          const float xv = s == 0 ? x[b].x : s == 1 ? x[b].y : s == 2 ? x[b].z : x[b].w;
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(ws[c], xv, acc[c][b], 0, 0, 0);
        }
      }
    };
#pragma unroll
    for (int p = 0; p < kPF; ++p) load(p, p);
    int j = 0;
    for (; j + NB <= nch; j += NB) {
#pragma unroll
      for (int p = 0; p < NB; ++p) {
        load((p + kPF) % NB, j + p + kPF);
        mma(p, j + p);
      }
    }
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      if (j + p < nch) {
        load((p + kPF) % NB, j + p + kPF);
        mma(p, j + p);
      }
    }
  }
  // value r of block (c, b): column n0 + 4(4 lq + r) + c, row m = 16 b + li
  float* pt = P + (long long)blockIdx.y * M * N;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * b + li, n = n0 + 4 * (4 * lq + r) + c;
        if (m < M && n < N) pt[(long long)m * N + n] = acc[c][b][r];
      }
}

// C[m][n] = sum over splits s, in split order, of P[s][m][n]; one thread per
// output element (measured faster than float4-per-thread variants here: the
// partials were just written by other XCDs and the loads are latency-bound).
__global__ __launch_bounds__(256) void sgemm_skinny_reduce(int M, int N, const float* __restrict__ P,
                                                           int splits, float* __restrict__ C, int ldc) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)M * N) return;
  const long long ps = (long long)M * N;
  float s = 0.f;
  for (int sp = 0; sp < splits; ++sp) s += P[sp * ps + t];
  C[(t / N) * ldc + t % N] = s;
}

bool use_fma(int m) { return m <= 4; }

int mma_mb(int m) { return m <= 16 ? 1 : 2; }

// k rows per split and split count.  The FMA path splits k 16 ways
// (measured best at K 4096 / N 11008); the MFMA path stages its A slice in
// LDS, which bounds the rows per split by the staging registers, and keeps
// ~2 workgroups per CU.
void plan(int m, int n, int k, int* kchunk, int* splits) {
  if (use_fma(m)) {
    int s = 16;
    if (k < 16 * 4 * kFmaUnroll) s = (k + 4 * kFmaUnroll - 1) / (4 * kFmaUnroll);
    if (s < 1) s = 1;
    int kc = (k + s - 1) / s;
    *kchunk = kc;
    *splits = (k + kc - 1) / kc;
    return;
  }
  const int mb = mma_mb(m);
  const int max_rows = kStageF4 * 256 * 4 / (16 * mb);  // staged A^T fits the unrolled loads
  const int colgroups = (n + kMmaCols - 1) / kMmaCols;
  int s = (512 + colgroups - 1) / colgroups;
  int kc = (k + s - 1) / s;
  kc = (kc + 15) / 16 * 16;
  if (kc > max_rows) kc = max_rows;
  *kchunk = kc;
  *splits = (k + kc - 1) / kc;
}

}  // namespace

namespace bch {

size_t sgemm_skinny_workspace_bytes(int m, int n, int k) {
  int kc, s;
  plan(m, n, k, &kc, &s);
  return sizeof(float) * (size_t)s * (size_t)m * (size_t)n;
}

bool sgemm_skinny_applies(int m, int n, int k, const float* A, int lda, const float* B, int ldb) {
  (void)A;
  (void)lda;
  if (m < 1 || m > 32 || n < 4 || k < 1) return false;
  if (n % 4 != 0 || ldb % 4 != 0) return false;
  if (B && (reinterpret_cast<uintptr_t>(B) & 15) != 0) return false;
  return true;
}

const char* sgemm_skinny_kernel_name(int m) {
  if (use_fma(m)) return "sgemm_skinny_fma";
  return mma_mb(m) == 1 ? "sgemm_skinny_mfma<1>" : "sgemm_skinny_mfma<2>";
}

hipError_t launch_sgemm_skinny(hipStream_t s, int m, int n, int k, const float* A, int lda,
                               const float* B, int ldb, float* C, int ldc, void* ws, size_t ws_bytes) {
  int kchunk, splits;
  plan(m, n, k, &kchunk, &splits);
  if (ws == nullptr || ws_bytes < sgemm_skinny_workspace_bytes(m, n, k)) return hipErrorInvalidValue;
  float* P = static_cast<float*>(ws);
  if (use_fma(m)) {
    dim3 grid((n + kFmaCols - 1) / kFmaCols, splits), block(256);
    if (m == 1)
      hipLaunchKernelGGL(sgemm_skinny_fma<1>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
    else if (m == 2)
      hipLaunchKernelGGL(sgemm_skinny_fma<2>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
    else
      hipLaunchKernelGGL(sgemm_skinny_fma<4>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
  } else {
    dim3 grid((n + kMmaCols - 1) / kMmaCols, splits), block(256);
    const int mb = mma_mb(m);
    const size_t lds = sizeof(float) * 16 * mb * (size_t)(kchunk + 4);
    const int avec = (lda % 4 == 0) && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
    if (mb == 1) {
      static bool set1 = false;
      if (!set1) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(sgemm_skinny_mfma<1>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(sizeof(float) * 16 * 1 * (kStageF4 * 256 * 4 / (16 * 1) + 4)));
        if (e != hipSuccess) return e;
        set1 = true;
      }
      hipLaunchKernelGGL(sgemm_skinny_mfma<1>, grid, block, lds, s, m, n, k, A, lda, B, ldb, P, kchunk, avec);
    } else {
      static bool set2 = false;
      if (!set2) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(sgemm_skinny_mfma<2>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(sizeof(float) * 16 * 2 * (kStageF4 * 256 * 4 / (16 * 2) + 4)));
        if (e != hipSuccess) return e;
        set2 = true;
      }
      hipLaunchKernelGGL(sgemm_skinny_mfma<2>, grid, block, lds, s, m, n, k, A, lda, B, ldb, P, kchunk, avec);
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long total = (long long)m * n;
  hipLaunchKernelGGL(sgemm_skinny_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, m, n, P,
                     splits, C, ldc);
  return hipGetLastError();
}

}  // namespace bch
