// sgemm_skinny.hip -- decode-shaped f32 GEMM (m <= 32) for gfx950.
//
// Replaces the K3 path of MatMul::execute (crates/barracuda/src/ops/
// matmul.rs:65-74 routes m < 256 to shaders/math/matmul_tiled_f64.wgsl,
// where for m <= 32 most of each 16x16 workgroup holds padding rows) for
// small m.  Contract unchanged: C[m,n] = sum_p A[m,p] B[p,n], f32.
//
// The job is streaming B ([k, n] row-major, k*n*4 bytes) from HBM once.
// The main kernels write split-k partials; a second kernel sums each
// output's partials in a fixed order, so results are deterministic.
//   * m <= 4, sgemm_skinny_fma: a wavefront owns 256 columns (lane l holds
//     columns 4l..4l+3, one 1 KB row segment per load); the four wavefronts
//     of a workgroup take interleaved rows with 8 row loads in flight; A[i][k]
//     is wave-uniform and comes through the scalar cache.  k is split 16 ways.
//   * 16 < m <= 32 (K % 4 == 0, aligned A), sgemm_skinny_w32: the same
//     stream-K layout with v_mfma_f32_32x32x2_f32 over all 32 rows at once,
//     512-byte row segments per load and one wave per SIMD (described at
//     the kernel).
//   * 4 < m <= 32 otherwise, sgemm_skinny_sk: at 2m multiply-adds per B element the
//     non-packed FP32 VALU cannot keep up with HBM, so v_mfma_f32_16x16x4_f32
//     computes C^T = B^T A^T (m padded to 16 or 32).  The work is cut into
//     units of 16 rows x 256 columns (4 wavefronts x 64 columns), ordered
//     column group by column group, and every workgroup takes an equal
//     contiguous run of units (stream-K): with one workgroup per CU every
//     CU streams the same number of bytes.  A run crosses at most a few
//     column-group boundaries; each run segment leaves one partial block.
//     In a unit, lane l = 16q + i loads float4 B[k][n0 + 4i .. +3] and feeds
//     component c to MFMA block c; lane quarter q takes rows 4q + s in step s.
//     The A^T operand of a unit is one float4 of A per lane, loaded from
//     L2 with the unit's B (A aligned; otherwise the workgroup's A^T slice
//     is staged in LDS once); B loads run PF units ahead of the MFMAs.
//   * Measured on MI355X (K 4096, N 11008, weights rotated past the 256 MB
//     Infinity Cache): the stream-K layout removes the tail of an uneven
//     grid (516 workgroups on 256 CUs); kernel code is kept small (one
//     unrolled pipeline step, rolled staging), as every CU fetches the whole
//     kernel from L2 once per launch.  An in-kernel "last workgroup reduces"
//     (256 workgroups, 43 column groups, 32 KB partial blocks) measured 3-9 us
//     per call for the agent-scope release/acquire alone, and the last
//     workgroup of a group then reads every slot by itself, so the reduction
//     stays a separate launch.  A full-K column-strip layout (no partials,
//     one launch) uses only N / 64 = 172 CUs and streamed at 5.2 TB/s.
#include "bch_internal.h"

#include <stdint.h>

#include <algorithm>
#include <atomic>


namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kFmaCols = 256;  // columns per workgroup, FMA kernel
constexpr int kFmaUnroll = 8;
constexpr int kFmaSplits = 16;
constexpr int kSkCols = 256;   // columns per unit / column group (4 x 64)
constexpr int kSkRows = 16;    // rows per unit
constexpr int kSkPF = 3;       // units of B in flight ahead of the MFMAs
constexpr int kLdsBytes = 160 * 1024;

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

// C[m][n] = sum over splits s < splits, in split order, of P[s][m][n].  The
// loads of a batch of 16 partials are all in flight before the adds.  Then
// the linear layer's epilogue: + bias[n], then the activation (both optional).
__device__ __forceinline__ float epilogue(float s, const float* __restrict__ bias, int n, int act) {
  if (bias) s += bias[n];
  return bch::activate(s, act);
}

// Block (x, m) covers columns 256 x .. 256 x + 255 of row m.
__global__ __launch_bounds__(256) void sgemm_skinny_reduce(int M, int N, const float* __restrict__ P, int splits,
                                                           float* __restrict__ C, int ldc,
                                                           const float* __restrict__ bias, int act) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const long long t = (long long)m * N + n;
  const long long ps = (long long)M * N;
  float s = 0.f;
  for (int i = 0; i < splits; i += 16) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = P[(long long)min(i + q, splits - 1) * ps + t];
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (i + q < splits) s += v[q];
  }
  C[(long long)m * ldc + n] = epilogue(s, bias, n, act);
}

// ---------------------------------------------------------------- 4 < m <= 32
// Stream-K unit bookkeeping: U units, G workgroups, workgroup w owns units
// [w U / G, (w + 1) U / G).  The workgroup holding unit u:
__host__ __device__ inline int wg_of_unit(long long u, long long U, int G) { return (int)(((u + 1) * G - 1) / U); }

// Partial block of (column group g, slot s): P[((g * smax + s) * M + m) * 256 + column - 256 g], the slot
// being the workgroup's position among those covering g.  AREG (lda % 4 == 0,
// K % 4 == 0, A 16-byte aligned): the MFMA's A^T operand is one float4 of A
// per lane per unit and block, loaded with that unit's B and from L2 (A is
// small and shared by every workgroup), PF units ahead like B.  Otherwise the
// workgroup's A^T slice is staged in LDS once with scalar loads.  Measured at
// K 4096, N 11008, M 8: staging the slice with direct-to-LDS loads before the
// first MFMA cost 1.7 us per call over the register operand.
template <int MB, bool AREG>
__global__ __launch_bounds__(256, 1) void sgemm_skinny_sk(int M, int N, int K, const float* __restrict__ A,
                                                          int lda, const float* __restrict__ B, int ldb,
                                                          float* __restrict__ P, long long U, int G, int kb,
                                                          int smax) {
  extern __shared__ float4 smem4[];
  float* xs = reinterpret_cast<float*>(smem4);  // A^T (staged path): [16 MB][16 nu + 4]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane >> 4, li = lane & 15;
  const int w = blockIdx.x;
  const long long ub = (long long)w * U / G, ue = (long long)(w + 1) * U / G;
  const int nu = (int)(ue - ub);
  const int g0 = (int)(ub / kb), t0 = (int)(ub - (long long)g0 * kb);
  const int q4 = 4 * nu;  // float4 per staged row
  const int ldu = 4 * q4 + 4;
  constexpr int PF = kSkPF, NB = kSkPF + 1;

  const float* arow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) arow[b] = A + (long long)min(16 * b + li, M - 1) * lda;

  // B cursor: unit (lg, lt); advanced once per load, held at the last unit.
  float4 wv[NB][4];
  float4 av[NB][MB];
  int lg = g0, lt = t0, lcount = 0;
  auto load = [&](int sb) {
    const float* bp = B + min(lg * kSkCols + 64 * wave + 4 * li, N - 4);
    const int r0 = kSkRows * lt + 4 * lq;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      wv[sb][s] = bch::load_nt(reinterpret_cast<const float4*>(bp + (long long)min(r0 + s, K - 1) * ldb));
    if (AREG) {
      // A[16 b + li][r0 .. r0 + 3]: K % 4 == 0, so the float4 lies wholly below K or wholly past it
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        av[sb][b] = *reinterpret_cast<const float4*>(arow[b] + min(r0, K - 4));
        if (r0 >= K) av[sb][b] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    ++lcount;  // uniform arithmetic, no branch between the loads
    lt += lcount < nu ? 1 : 0;
    const int wrap = lt == kb ? 1 : 0;
    lt -= wrap * kb;
    lg += wrap;
  };

  if (AREG) {
#pragma unroll
    for (int p = 0; p < PF; ++p) load(p);
  } else {
    // k of staged float4 q (its unit is t0 + q / 4, wrapped into the next column group)
    auto k_of = [&](int q) {
      int t = t0 + (q >> 2);
      while (t >= kb) t -= kb;
      return kSkRows * t + 4 * (q & 3);
    };
    for (int e = tid; e < 16 * MB * q4; e += 256) {
      const int m = e / q4, q = e - m * q4;
      const int k = k_of(q);
      const float* ar = A + (long long)min(m, M - 1) * lda;
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = m < M && k + c < K ? ar[k + c] : 0.f;
      *reinterpret_cast<float4*>(xs + m * ldu + 4 * q) = make_float4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int p = 0; p < PF; ++p) load(p);
    __syncthreads();
  }

  f32x4v acc[4][MB];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[c][b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  int gcur = g0, tcur = t0;
  int slot = w - wg_of_unit((long long)g0 * kb, U, G);  // later groups start in this workgroup: slot 0
  // value r of block (c, b) is column 64 wave + 16 lq + 4 r + c, row 16 b + li: a float4 over c
  auto flush = [&]() {
    float* pt = P + (long long)(gcur * smax + slot) * M * kSkCols + 64 * wave + 16 * lq;
    const int nrem = N - gcur * kSkCols - 64 * wave - 16 * lq;
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = 16 * b + li;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (m < M && 4 * r < nrem)
          *reinterpret_cast<float4*>(pt + m * kSkCols + 4 * r) =
              make_float4(acc[0][b][r], acc[1][b][r], acc[2][b][r], acc[3][b][r]);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c][b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
    }
  };
  auto mma = [&](int sb, int i) {
    float4 x[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b)
      x[b] = AREG ? av[sb][b] : *reinterpret_cast<const float4*>(xs + (16 * b + li) * ldu + 16 * i + 4 * lq);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float ws[4] = {wv[sb][s].x, wv[sb][s].y, wv[sb][s].z, wv[sb][s].w};
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const float xv = s == 0 ? x[b].x : s == 1 ? x[b].y : s == 2 ? x[b].z : x[b].w;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(ws[c], xv, acc[c][b], 0, 0, 0);
      }
    }
  };
  // one unrolled copy of the pipeline step: loads are unconditional (the
  // cursor holds at the last unit), the MFMAs are guarded by i < nu
  for (int i = 0; i < nu; i += NB) {
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      load((p + PF) % NB);
      if (i + p < nu) {
        mma(p, i + p);
        if (++tcur == kb && i + p + 1 < nu) {
          flush();
          tcur = 0;
          ++gcur;
          slot = 0;
        }
      }
    }
  }
  flush();
}

// ---------------------------------------------------------------- 16 < m <= 32
// v_mfma_f32_32x32x2_f32 computes C^T = B^T A^T with all 32 rows of A in one
// tile, so each B element feeds exactly one MFMA.  A workgroup is 4 waves:
// column half ch = wave & 1 (128 of the group's 256 columns) and row stream
// rs = wave >> 1.  A unit is 32 rows x 256 columns; stream rs takes rows
// 16 rs .. 16 rs + 15 of it as 8 row pairs (p, p + 8), lane half lh holding
// row 8 lh + p.  One float4 load per pair gives lane (lh, j) the columns
// 4j .. 4j + 3 of its row, i.e. the MFMA A-operand of column block c = 0..3
// (columns {4j + c}): no shuffles, 512 contiguous bytes per row per load.
// A is read as two float4 per lane per unit (A[m][r0 .. r0 + 7], m = lane
// & 31), straight from L2.  The loads are branch-free (a fixed 10 per unit)
// so the compiler's wait on a unit's data leaves the PF later units in
// flight.  With the MFMA accumulators in VGPRs (this file is built with
// -mllvm -amdgpu-mfma-vgpr-form) nothing is copied to AGPRs in the loop.
// At a flush the two row streams are summed through LDS, in stream order.
// The dynamic LDS request (kW32Lds) keeps one workgroup per CU, so every
// SIMD runs exactly one wave: two waves on one SIMD would share its matrix
// core, and with 64 MACs per B element the MFMA time is close to the HBM
// time.  One unit of loads in flight ahead of the MFMAs (PF = 1) measured
// fastest at K 4096, N 11008 (PF 1 / 2 / 3: 37.7 / 38.7 / 40 us per launch):
// deeper prefetch buys no bandwidth and costs registers.  Requires K % 4 == 0,
// lda % 4 == 0 and 16-byte aligned A (the clamped float4 A loads stay inside
// the row).
constexpr int kW32Rows = 32;
constexpr int kW32PF = 1;
constexpr int kW32Lds = 96 * 1024;  // > half of the CU's 160 KB: one workgroup per CU

template <int PF, bool EDGE, int MB = 1>
__global__ __launch_bounds__(256, 1) void sgemm_skinny_w32(int M, int N, int K, const float* __restrict__ A, int lda,
                                                           const float* __restrict__ B, int ldb,
                                                           float* __restrict__ P, long long U, int G, int nblk,
                                                           int smax) {
  typedef float f32x16v __attribute__((ext_vector_type(16)));
  extern __shared__ float4 smem4[];
  constexpr int LDR = 128 + 4;
  float* red = reinterpret_cast<float*>(smem4);  // [2 column halves][32 MB m][LDR]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ch = wave & 1, rs = wave >> 1;
  const int lh = lane >> 5, lm = lane & 31;
  const int w = blockIdx.x;
  const long long ub = (long long)w * U / G, ue = (long long)(w + 1) * U / G;
  const int nu = (int)(ue - ub);
  const int g0 = (int)(ub / nblk), t0 = (int)(ub - (long long)g0 * nblk);
  constexpr int NB = PF + 1;
  const float* arow[MB];  // row block rb: rows 32 rb + lm; rows m >= M compute columns never stored
#pragma unroll
  for (int rb = 0; rb < MB; ++rb) arow[rb] = A + (long long)min(32 * rb + lm, M - 1) * lda;

  float4 bv[NB][8];
  float4 av[NB][MB][2];
  int lg = g0, lt = t0, lcount = 0;  // load cursor: advanced once per load, held at the last unit
  auto load = [&](int sb) {
    const int col = min(lg * kSkCols + 128 * ch + 4 * lm, N - 4);
    const int r0 = kW32Rows * lt + 16 * rs + 8 * lh;
#pragma unroll
    for (int p = 0; p < 8; ++p)
      bv[sb][p] = bch::load_nt(reinterpret_cast<const float4*>(B + (long long)min(r0 + p, K - 1) * ldb + col));
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
      av[sb][rb][0] = *reinterpret_cast<const float4*>(arow[rb] + min(r0, K - 4));
      av[sb][rb][1] = *reinterpret_cast<const float4*>(arow[rb] + min(r0 + 4, K - 4));
    }
    if (EDGE) {  // rows past K (last unit when K % 32 != 0): zero both operands
#pragma unroll
      for (int p = 0; p < 8; ++p)
        if (r0 + p >= K) bv[sb][p] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int rb = 0; rb < MB; ++rb) {
        float* a = reinterpret_cast<float*>(&av[sb][rb][0]);
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (r0 + c >= K) a[c] = 0.f;
      }
    }
    ++lcount;
    lt += lcount < nu ? 1 : 0;
    const int wrap = lt == nblk ? 1 : 0;
    lt -= wrap * nblk;
    lg += wrap;
  };
  // The prologue units are issued in order (no interleaving across units):
  // the loop header's wait then only has to cover the oldest unit, as on the
  // back edge; interleaved, the last-issued load belongs to unit 0 and the
  // header's single wait becomes vmcnt(0) on every iteration.
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    load(p);
    __builtin_amdgcn_sched_barrier(0);
  }

  f32x16v acc[MB][4];
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][c][r] = 0.f;

  int gcur = g0, tcur = t0;
  int slot = w - wg_of_unit((long long)g0 * nblk, U, G);
  // value r of block c, row block rb: row m = 32 rb + lm, column 4 i + c of the wave's half,
  // i = 8 (r / 4) + 4 lh + r % 4
  auto flush = [&]() {
    float* rbuf = red + ch * 32 * MB * LDR;
    if (rs == 1) {
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
          *reinterpret_cast<float4*>(rbuf + (32 * rb + lm) * LDR + 4 * i) =
              make_float4(acc[rb][0][r], acc[rb][1][r], acc[rb][2][r], acc[rb][3][r]);
        }
    }
    __syncthreads();
    if (rs == 0) {
      const int nrem = N - gcur * kSkCols - 128 * ch;
#pragma unroll
      for (int rb = 0; rb < MB; ++rb) {
        const int m = 32 * rb + lm;
        if (m < M) {
          float* pt = P + (long long)(gcur * smax + slot) * M * kSkCols + 128 * ch + m * kSkCols;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
            const float4 o = *reinterpret_cast<const float4*>(rbuf + m * LDR + 4 * i);
            if (4 * i < nrem)
              *reinterpret_cast<float4*>(pt + 4 * i) =
                  make_float4(acc[rb][0][r] + o.x, acc[rb][1][r] + o.y, acc[rb][2][r] + o.z, acc[rb][3][r] + o.w);
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[rb][c][r] = 0.f;
  };
  auto mma = [&](int sb) {
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
      const float a8[8] = {av[sb][rb][0].x, av[sb][rb][0].y, av[sb][rb][0].z, av[sb][rb][0].w,
                           av[sb][rb][1].x, av[sb][rb][1].y, av[sb][rb][1].z, av[sb][rb][1].w};
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const float b4[4] = {bv[sb][p].x, bv[sb][p].y, bv[sb][p].z, bv[sb][p].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[rb][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(b4[c], a8[p], acc[rb][c], 0, 0, 0);
      }
    }
  };
  for (int i = 0; i < nu; i += NB) {
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      load((p + PF) % NB);
      if (i + p < nu) {
        mma(p);
        if (++tcur == nblk && i + p + 1 < nu) {
          flush();
          tcur = 0;
          ++gcur;
          slot = 0;
        }
      }
    }
  }
  flush();
}

// C[m][n] = sum of the partial blocks of n's column group, in slot order
// (the k order); loads in batches of 8, all in flight before the adds.
// Block (x, m) covers columns 256 x .. 256 x + 255 of row m; the partial
// block width is 1 << cshift columns.  The group's slot count comes from the
// stream-K bookkeeping in 32-bit arithmetic when U G < 2^32 (WIDE: 64-bit);
// 64-bit divisions per thread measured as most of the kernel's instructions.
template <bool WIDE>
__global__ __launch_bounds__(256) void sgemm_skinny_sk_reduce(int M, int N, const float* __restrict__ P, long long U,
                                                              int G, int kb, int smax, float* __restrict__ C,
                                                              int ldc, const float* __restrict__ bias, int act,
                                                              int cshift) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const int g = n >> cshift;
  int ns;
  if (WIDE) {
    ns = wg_of_unit((long long)g * kb + kb - 1, U, G) - wg_of_unit((long long)g * kb, U, G) + 1;
  } else {
    const unsigned u0 = (unsigned)g * (unsigned)kb, uu = (unsigned)U, gg = (unsigned)G;
    ns = (int)(((u0 + (unsigned)kb) * gg - 1u) / uu) - (int)(((u0 + 1u) * gg - 1u) / uu) + 1;
  }
  const float* p = P + ((long long)g * smax * M + m) * (1 << cshift) + (n - (g << cshift));
  const long long st = (long long)M << cshift;
  float s = 0.f;
  for (int i = 0; i < ns; i += 8) {
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = p[(long long)min(i + q, ns - 1) * st];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (i + q < ns) s += v[q];
  }
  C[(long long)m * ldc + n] = epilogue(s, bias, n, act);
}

// Launch the split-k reduce of a stream-K plan (cols: partial block width, a power of two).
hipError_t launch_sk_reduce(hipStream_t s, int m, int n, const float* P, long long U, int G, int kb, int smax,
                            float* C, int ldc, const float* bias, int act, int cols) {
  const dim3 grid((unsigned)((n + 255) / 256), (unsigned)m);
  const int cshift = __builtin_ctz((unsigned)cols);  // cols: a power of two
  if ((unsigned long long)U * (unsigned long long)G < (1ULL << 32))
    hipLaunchKernelGGL(sgemm_skinny_sk_reduce<false>, grid, dim3(256), 0, s, m, n, P, U, G, kb, smax, C, ldc, bias,
                       act, cshift);
  else
    hipLaunchKernelGGL(sgemm_skinny_sk_reduce<true>, grid, dim3(256), 0, s, m, n, P, U, G, kb, smax, C, ldc, bias,
                       act, cshift);
  return hipGetLastError();
}

// ---------------------------------------------------------------- transposed weights, 8 < m <= 32
// C[m][n] = sum_k A[m][k] W[n][k]: the linear layer with W [out, in]
// (shaders/misc/linear_f64.wgsl) at decode sizes (and m <= 8 when N is too
// narrow for the whole-row kernel below).  Stream-K over units of
// R = 16 RB rows of W (output columns n) x KU = 8192 / R k -- 32 KB of W --
// ordered row group by row group.  RB = 2 (32 x 256, every row one 1 KB
// piece) for m <= 16; RB = 4 (64 x 128) for m > 16, which halves the bytes of
// A read per byte of W (A's slice of a unit is m x KU).  Workgroups of 8
// wavefronts, one per CU:
//   * waves 4..7 copy units into a 3-slot LDS ring with direct-to-LDS loads
//     (global_load_lds_dwordx4, 8 per wave and unit, each one 1 KB row or two
//     512 B rows).  A slot holds its rows unpadded; the 16-byte chunks of row
//     r are XOR-swizzled by r % 8 through the loads' global addresses, so the
//     operand reads below are free of bank conflicts.  A loader waits for a
//     unit with s_waitcnt on its own load count;
//   * waves 0..3 run v_mfma_f32_16x16x4_f32 (C^T = W A^T on 16 n x 16 m
//     blocks, m padded to 16 or 32) over k quarters of each unit: lane
//     l = 16 q + i reads row i of a 16-row block at k = 16 t + 4 q .. + 3
//     from the ring and the same four k of A row 16 b + i from L2 (two units
//     ahead), and feeds k = 16 t + 4 q + c in step (t, c).
// One workgroup barrier per unit hands the ring over: the loaders wait for
// unit i + 1 before it, the MFMA waves read unit i + 1 after it, between the
// two halves of unit i's MFMAs (so the reads overlap MFMAs).  At the end of a
// run segment (the units of one row group in this workgroup) one more
// barrier hands the four waves' sums to LDS, where they are added in wave
// order.  A segment that covers its whole row group is stored to C with the
// epilogue.  Otherwise the group is split over consecutive workgroups and
// combined in this kernel, with no second launch:
//   * its owner is the last of them, whose first segment is the group's
//     tail; it keeps that block in registers until the end of its run;
//   * every other one (a contributor, whose last segment it is) stores its
//     block with agent-scope (sc1) stores, waits for their completion
//     (s_waitcnt vmcnt(0)) and then sets its flag to the launch's epoch;
//   * at the end of its run the owner waits for the flags of all its
//     contributors, then loads their blocks (sc1, up to four slots per
//     batch), adds them in k order followed by its own, applies the
//     epilogue, stores C and resets the flags.
// An owner waits only on lower-numbered workgroups, which are dispatched
// before it and never wait before storing their block, so the wait always
// ends; it is bounded anyway (LaunchCtl::spin polls, 2^22 by default, about
// 0.1 s): a block that never arrives turns the outputs NaN and sets the
// calling context's fault word, so the host reports a lost device at its
// next synchronisation instead of returning NaN silently.  The epoch (64-bit,
// one per launch) keeps stale flags from matching; the reset keeps a replay
// of a captured launch, which reuses its epoch, from matching the previous
// replay's flags (a contributor that sets its flag after its owner gave up
// could match a later replay's owner, but the context is lost by then).  EDGE (K % KU != 0): loads past
// K read from K - 4 and both MFMA operands of such k are zeroed where they
// are used; rows past N read row N - 1 and are never stored.  Requires
// K % 4 == 0, lda % 4 == 0, ldw % 4 == 0 and 16-byte aligned A and W.
// Measured on one MI355X at K 4096, N 11008, kernel alone (M = 8 / 32):
// 32 x 256 units padded to 260-float rows 30.9 / 45.7 us; swizzled 31.2 /
// 43.3 us; 64 x 128 swizzled 32.6 / 38.1 us.  With A's loads removed the
// padded kernel took 31.6 / 37.2 us: at m > 16 A's slice was as many bytes
// as the weights.  A pure read of the weights in this schedule takes 30.2
// us.  Whole-row ownership (each workgroup its own 43 rows over all K, no
// partials) measured 37.7 us at M = 8: the row blocks left per workgroup are
// short and keep too few bytes in flight.
constexpr int kRgUnit = 32768;  // bytes of W per unit and ring slot
constexpr int kRgD = 3;         // ring slots

template <int RB>
struct RgShape {
  static constexpr int R = 16 * RB;       // rows of W (output columns) per unit
  static constexpr int KU = 8192 / R;     // k per unit
  static constexpr int KQ = KU / 4;       // k per MFMA wave and unit
  static constexpr int TT = KQ / 16;      // 16-k steps per MFMA wave and unit
  static constexpr int RPI = 256 / KU;    // rows per load instruction
};

int rg_rb(int m) { return m <= 16 ? 2 : 4; }

template <int MB, int RB>
constexpr int rg_lds_bytes() {
  return kRgD * kRgUnit + 4 * RB * MB * 4 * 64 * 4;  // ring, then the segment-end sums of 4 waves
}

typedef __attribute__((address_space(3))) void lds_void;

// loader: wait until at most n of this wave's units (8 loads each) are in flight
__device__ __forceinline__ void rg_wait_units(int n) {
  if (n <= 0)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (n == 1)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

// workgroup barrier that no memory access or instruction is moved across
__device__ __forceinline__ void rg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maximum)
constexpr int kLgkmZero = 0xC07F;


template <int MB, int RB, bool EDGE>
__global__ __launch_bounds__(512, 1) void sgemm_skinny_nt_ring(
    int M, int N, int K, const float* __restrict__ A, int lda, const float* __restrict__ W, int ldw,
    float* __restrict__ C, int ldc, const float* __restrict__ bias, int act, float* __restrict__ P,
    unsigned long long* __restrict__ F, unsigned long long epoch, long long U, int G, int nkb, int smax,
    unsigned* __restrict__ fault, unsigned spin) {
  using S = RgShape<RB>;
  constexpr int R = S::R, KU = S::KU, KQ = S::KQ, TT = S::TT, RPI = S::RPI;
  extern __shared__ float4 smem4[];
  char* ring = reinterpret_cast<char*>(smem4);
  float* red = reinterpret_cast<float*>(ring + kRgD * kRgUnit);  // [4 waves][RB rb][MB][4 r][64 lanes]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int w = blockIdx.x;
  const long long ub = (long long)w * U / G, ue = (long long)(w + 1) * U / G;
  const int nu = (int)(ue - ub);  // >= 1: G <= U
  const int g0 = (int)(ub / nkb), t0 = (int)(ub - (long long)g0 * nkb);

  if (wave >= 4) {
    // ---- loader wave lw: rows 4 RB lw .. 4 RB lw + 4 RB - 1 of every unit, RPI rows per load
    const int lw = wave - 4;
    const int lrow = lane / (64 / RPI), chunk = lane % (64 / RPI);  // this lane's row in a load, its chunk slot
    int lg = g0, lt = t0;
    auto issue = [&](int i) {
      char* dst = ring + (i % kRgD) * kRgUnit;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int rl = 4 * RB * lw + RPI * j;  // first row of load j
        const int row = rl + lrow;
        int k = KU * lt + 4 * (chunk ^ (row & 7));
        if (EDGE) k = min(k, K - 4);
        const float* src = W + (long long)min(R * lg + row, N - 1) * ldw + k;
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(dst + rl * KU * 4), 16, 0, 2 /* nt */);
      }
      if (++lt == nkb) {
        lt = 0;
        ++lg;
      }
    };
    const int n0 = nu < kRgD - 1 ? nu : kRgD - 1;
    for (int i = 0; i < n0; ++i) issue(i);
    rg_wait_units(n0 - 1);
    __builtin_amdgcn_s_barrier();
    int st = t0;
    for (int i = 0; i < nu; ++i) {
      if (i + kRgD - 1 < nu) issue(i + kRgD - 1);
      const int last = i + kRgD - 1 < nu ? i + kRgD - 1 : nu - 1;
      rg_wait_units(last - (i + 1));  // unit i + 1 has landed
      __builtin_amdgcn_s_barrier();
      const bool group_end = ++st == nkb;
      if (group_end) st = 0;
      if (group_end || i + 1 == nu) __builtin_amdgcn_s_barrier();  // the segment-end sums
    }
    return;
  }

  // ---- MFMA wave cw: k quarter [KQ cw, KQ cw + KQ) of every unit
  const int cw = wave, q = lane >> 4, i16 = lane & 15;
  const float* arow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) arow[b] = A + (long long)min(16 * b + i16, M - 1) * lda;
  constexpr int PX = 2, NX = PX + 1;  // units of A in flight ahead of the MFMAs
  float4 av[NX][MB][TT];
  int xt = t0, xn = 0;  // A cursor: advanced once per load, held at the last unit
  auto load_a = [&](int sb) {
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        int k = KU * xt + KQ * cw + 16 * tt + 4 * q;
        if (EDGE) k = min(k, K - 4);  // zeroed where used
        av[sb][b][tt] = *reinterpret_cast<const float4*>(arow[b] + k);
      }
    if (++xn < nu && ++xt == nkb) xt = 0;
  };
#pragma unroll
  for (int p = 0; p < PX; ++p) load_a(p);
  float4 wv[2][RB][TT];
  auto read_w = [&](int sb, int i) {
    const char* sl = ring + (i % kRgD) * kRgUnit;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int row = 16 * rb + i16, c = (KQ / 4) * cw + 4 * tt + q;
        wv[sb][rb][tt] = *reinterpret_cast<const float4*>(sl + row * KU * 4 + ((c ^ (row & 7)) << 4));
      }
  };
  f32x4v acc[RB][MB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[rb][b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  // half h (steps [h TT / 2, (h + 1) TT / 2)) of the unit whose k starts at kbase
  auto mma = [&](int sw, int sx, int h, int kbase) {
#pragma unroll
    for (int tt = h * TT / 2; tt < (h + 1) * TT / 2; ++tt) {
      const bool live = !EDGE || kbase + KQ * cw + 16 * tt + 4 * q < K;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          const float4 a4 = av[sx][b][tt];
          float x = c == 0 ? a4.x : c == 1 ? a4.y : c == 2 ? a4.z : a4.w;
          if (EDGE) x = live ? x : 0.f;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const float4 w4 = wv[sw][rb][tt];
            float y = c == 0 ? w4.x : c == 1 ? w4.y : c == 2 ? w4.z : w4.w;
            if (EDGE) y = live ? y : 0.f;
            acc[rb][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(y, x, acc[rb][b], 0, 0, 0);
          }
        }
    }
  };
  // Segment end: value r of block (rb, b) at lane (q, i) is n = 16 rb + 4 q + r,
  // m = 16 b + i.  After the exchange wave cw holds the sums of column n = lane % R
  // for rows m = cw + 4 (u 4 / RB + lane / R), u < MB RB.
  // Partial block of (group g, slot sl): [sl][wave][u][lane] floats, lane-major.
  constexpr int NV = MB * RB;  // sums per lane
  __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(P, 0, 0x7fffffff, 0x00020000);
  auto pofs = [&](int g, int sl, int u) { return ((((g * smax + sl) * 4 + cw) * NV + u) * 64 + lane) * 4; };
  const int ncol = lane % R;
  auto row_of = [&](int u) { return cw + 4 * (u * (4 / RB) + lane / R); };
  float keep[NV];
  int own_g = -1;
  auto store_c = [&](int g, const float* val) {
    const int n = R * g + ncol;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int m = row_of(u);
      if (m < M && n < N) C[(long long)m * ldc + n] = epilogue(val[u], bias, n, act);
    }
  };
  auto seg_end = [&](int g, long long a, long long b) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int bb = 0; bb < MB; ++bb)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(((cw * RB + rb) * MB + bb) * 4 + r) * 64 + lane] = acc[rb][bb][r];
    __builtin_amdgcn_s_waitcnt(kLgkmZero);
    rg_barrier();
    const int rb = ncol >> 4, qq = (ncol >> 2) & 3, r = ncol & 3;
    constexpr int kWave = RB * MB * 4 * 64;  // one wave's values
    float val[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int m = row_of(u);
      const int e = ((rb * MB + (m >> 4)) * 4 + r) * 64 + 16 * qq + (m & 15);
      val[u] = ((red[e] + red[kWave + e]) + red[2 * kWave + e]) + red[3 * kWave + e];
    }
    const long long gs = (long long)g * nkb, ge = gs + nkb;
    if (a == gs && b == ge) {
      store_c(g, val);
    } else if (b == ge) {
#pragma unroll
      for (int u = 0; u < NV; ++u) keep[u] = val[u];
      own_g = g;
    } else {
      const int sl = w - wg_of_unit(gs, U, G);
#pragma unroll
      for (int u = 0; u < NV; ++u)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val[u]), prs, pofs(g, sl, u), 0, 16 /* sc1 */);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane == 0)
        __hip_atomic_store(F + ((long long)g * smax + sl) * 4 + cw, epoch, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int rb2 = 0; rb2 < RB; ++rb2)
#pragma unroll
      for (int bb = 0; bb < MB; ++bb) acc[rb2][bb] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  };
  __builtin_amdgcn_s_barrier();  // unit 0 has landed
  asm volatile("" ::: "memory");
  read_w(0, 0);
  int gcur = g0, tcur = t0;
  long long seg_a = ub;  // first unit of the current run segment
  // unrolled 2 NX times so that both register rings are indexed statically
  for (int i0 = 0; i0 < nu; i0 += 2 * NX) {
#pragma unroll
    for (int p = 0; p < 2 * NX; ++p) {
      const int i = i0 + p;
      if (i < nu) {
        load_a((p + PX) % NX);
        mma(p & 1, p % NX, 0, KU * tcur);
        __builtin_amdgcn_s_waitcnt(kLgkmZero);  // this unit's ring reads are complete
        rg_barrier();
        if (i + 1 < nu) read_w((p + 1) & 1, i + 1);
        mma(p & 1, p % NX, 1, KU * tcur);
        const bool group_end = ++tcur == nkb;
        if (group_end || i + 1 == nu) {
          seg_end(gcur, seg_a, ub + i + 1);
          seg_a = ub + i + 1;
        }
        if (group_end) {
          tcur = 0;
          ++gcur;
        }
      }
    }
  }
  if (own_g >= 0) {
    // the contributors' blocks in k order, then this workgroup's own (the group's tail)
    const int nprev = w - wg_of_unit((long long)own_g * nkb, U, G);
    unsigned long long* fl = F + (long long)own_g * smax * 4 + cw;
    bool ok = true;
    float sum[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) sum[u] = 0.f;
    // every flag first, then the blocks in batches of up to four slots (one round trip each)
    for (int sl = 0; sl < nprev; ++sl) {
      unsigned n = 0;
      while (__hip_atomic_load(fl + 4 * sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch && n < spin) {
        __builtin_amdgcn_s_sleep(1);
        ++n;
      }
      ok = ok && n < spin;
    }
    // a block that never arrived: the outputs become NaN and the context's
    // fault word (pinned host memory) is set, which the host reports as a
    // lost device at its next synchronisation
    if (!ok && lane == 0 && fault != nullptr)
      __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    for (int s0 = 0; s0 < nprev; s0 += 4) {
      float v[4][NV];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int sl = min(s0 + j, nprev - 1);  // past the last slot: loaded again, not added
#pragma unroll
        for (int u = 0; u < NV; ++u)
          v[j][u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(prs, pofs(own_g, sl, u), 0, 16 /* sc1 */));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < NV; ++u)
          if (s0 + j < nprev) sum[u] += v[j][u];
    }
#pragma unroll
    for (int u = 0; u < NV; ++u) sum[u] = ok ? sum[u] + keep[u] : __builtin_nanf("");
    store_c(own_g, sum);
    if (lane == 0)
      for (int sl = 0; sl < nprev; ++sl) __hip_atomic_store(fl + 4 * sl, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- transposed weights, m <= 8, whole rows
// C[m][n] = sum_k A[m][k] W[n][k] with every workgroup owning whole rows of W
// (a contiguous run of output columns) over all of K: one launch, no split-k
// partials in HBM, no reduce kernel.  Rows of W are contiguous, so workgroup
// g streams rows [g N / G, (g + 1) N / G) as one contiguous block of memory.
// K is taken in passes of 4096; in a pass wave w owns k = 4096 p + 512 w ..
// + 511 of every row of the block, as two 1 KB loads per row (lane l holds
// k = 4096 p + 512 w + 256 j + 4 l .. + 3 of load j), so the eight waves
// read each row together, 16 KB contiguous, one row ahead of the FMAs.  The
// A values a lane multiplies are the same for every row: they sit in
// registers for the whole pass (MT x 8 floats), so a W float4 costs 4 MT
// FMAs and nothing else.  At the end of a row each lane folds its float4 of
// sums per row of A to one value; the 64 lane values of a (row, m) are summed
// in batches of 64 / MT rows through a per-wave LDS transpose (row stride 65
// floats, conflict-free both ways): each lane writes its MT values, then
// lane i adds the 64 values of (row, m) number i in a fixed order, which
// costs about two instructions per (row, m) against some twelve for a
// wavefront all-reduce.  The eight waves' k-slices of a row meet in LDS
// (part[row][wave][m], accumulated over the passes) and are added in wave
// order after the last pass, then the epilogue (+ bias[n], activation) is
// applied and C stored.  Results are deterministic.  EDGE: K is not a
// multiple of 4096, so loads past K are clamped and zeroed (a wave whose
// whole slice lies past K loads nothing).  Requires K % 4 == 0,
// lda % 4 == 0, ldw % 4 == 0 and 16-byte aligned A and W; the host keeps
// every block at or below kRowCap(MT) rows (more workgroups than CUs for a
// very wide N).
// Measured at K 4096, N 11008, per call (M = 1 / 2 / 4 / 5 / 8): 28.7 /
// 28.8 / 29.7 / 31.0 / 31.4 us.  Splitting K four ways over two row sets
// (A in 16 MT registers per lane): 29.3 / - / 30.6 / - / 32.3 us; two rows
// ahead 29.2 / 29.6 / 30.2 / - / 31.9 us.  The kernel it replaced (A staged
// in LDS, each wave streaming whole rows, one ds_read_b128 of A per W float4
// and row of A) took 29.4 / 30.7 / 31.8 us at M = 1 / 2 / 4, and 38.7 us at
// M = 8, where the LDS reads of A carried eight times the bytes of W.  At
// M = 16 (16 FMAs per W element) this layout is VALU-bound: 40 us, so
// m > 8 takes the ring kernel.
constexpr int kRowWaves = 8;                               // wavefronts per workgroup (one workgroup per CU)
constexpr int kRowPass = 4096;                             // k per pass
constexpr int kRowNJ = kRowPass / 256 / kRowWaves;         // 1 KB loads per wave and row
constexpr int kRowTS = 65;                                 // transpose row stride (floats)
constexpr int kRowRed = kRowWaves * 64 * kRowTS;           // floats of the transpose buffers
// rows per workgroup whose part[] fits next to the transpose buffers
constexpr int kRowCap(int mt) { return (kLdsBytes / 4 - kRowRed) / (kRowWaves * mt); }

template <int MT, bool EDGE>
__global__ __launch_bounds__(64 * kRowWaves, 1) void sgemm_skinny_nt_rows(int M, int N, int K,
                                                                         const float* __restrict__ A, int lda,
                                                                         const float* __restrict__ W, int ldw,
                                                                         float* __restrict__ C, int ldc,
                                                                         const float* __restrict__ bias,
                                                                         int act) {
  constexpr int RB = 64 / MT;  // rows per transpose batch
  extern __shared__ float4 smem4[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* red = reinterpret_cast<float*>(smem4) + wave * 64 * kRowTS;  // this wave's [64 values][kRowTS]
  float* part = reinterpret_cast<float*>(smem4) + kRowRed;            // [rows][kRowWaves][MT]
  const int r0 = (int)((long long)blockIdx.x * N / gridDim.x);
  const int r1 = (int)((long long)(blockIdx.x + 1) * N / gridDim.x);
  const int nr = r1 - r0;
  const int npass = (K + kRowPass - 1) / kRowPass;
  constexpr int PF = 1, NB = 2;

  for (int pass = 0; pass < npass; ++pass) {
    const int kw = kRowPass * pass + 256 * kRowNJ * wave;  // first k of this wave's slice
    const bool live = !EDGE || kw < K;                      // wave-uniform: the slice reaches below K
    const int kl = kw + 4 * lane;
    float4 a[MT][kRowNJ];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float* ar = A + (long long)min(m, M - 1) * lda;
#pragma unroll
      for (int j = 0; j < kRowNJ; ++j) {
        const int k = kl + 256 * j;
        float4 v = *reinterpret_cast<const float4*>(ar + (EDGE ? min(k, K - 4) : k));
        if (m >= M || (EDGE && k >= K)) v = make_float4(0.f, 0.f, 0.f, 0.f);
        a[m][j] = v;
      }
    }
    float4 wv[NB][kRowNJ];
    int lrow = 0;  // load cursor, held at the last row
    auto load = [&](int sb) {
      const float* wr = W + (long long)(r0 + lrow) * ldw;
#pragma unroll
      for (int j = 0; j < kRowNJ; ++j) {
        const int k = kl + 256 * j;
        if (live) {
          wv[sb][j] = bch::load_nt(reinterpret_cast<const float4*>(wr + (EDGE ? min(k, K - 4) : k)));
          if (EDGE && k >= K) wv[sb][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
          wv[sb][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      lrow += lrow + 1 < nr ? 1 : 0;
    };
    if (nr > 0) load(0);
    for (int i = 0; i < nr; i += NB) {
#pragma unroll
      for (int p = 0; p < NB; ++p) {
        load((p + PF) % NB);
        __builtin_amdgcn_sched_barrier(0);  // the next row's loads stay ahead of this row's FMAs
        const int row = i + p;
        if (row < nr) {
          float s[MT];
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int j = 0; j < kRowNJ; ++j) {
              acc.x = fmaf(a[m][j].x, wv[p][j].x, acc.x);
              acc.y = fmaf(a[m][j].y, wv[p][j].y, acc.y);
              acc.z = fmaf(a[m][j].z, wv[p][j].z, acc.z);
              acc.w = fmaf(a[m][j].w, wv[p][j].w, acc.w);
            }
            s[m] = (acc.x + acc.y) + (acc.z + acc.w);
          }
          const int b = row % RB;
#pragma unroll
          for (int m = 0; m < MT; ++m) red[(b * MT + m) * kRowTS + lane] = s[m];
          if (b == RB - 1 || row == nr - 1) {
            // this wave's LDS writes are complete before any lane reads them, and the reads before
            // the next batch overwrites them (one wave: no workgroup barrier)
            __builtin_amdgcn_s_waitcnt(kLgkmZero);
            __builtin_amdgcn_wave_barrier();
            if (lane < (b + 1) * MT) {
              const float* src = red + lane * kRowTS;
              float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
#pragma unroll
              for (int q = 0; q < 64; q += 4) {
                t0 += src[q];
                t1 += src[q + 1];
                t2 += src[q + 2];
                t3 += src[q + 3];
              }
              const float v = (t0 + t1) + (t2 + t3);
              float* dst = part + ((row - b + lane / MT) * kRowWaves + wave) * MT + lane % MT;
              *dst = pass == 0 ? v : *dst + v;
            }
            __builtin_amdgcn_s_waitcnt(kLgkmZero);
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < nr * M; e += 64 * kRowWaves) {
    const int m = e / nr, row = e - m * nr;
    const float* pr = part + row * kRowWaves * MT + m;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kRowWaves; ++w) v += pr[w * MT];
    C[(long long)m * ldc + r0 + row] = epilogue(v, bias, r0 + row, act);
  }
}

bool use_fma(int m) { return m <= 4; }

int sk_mb(int m) { return m <= 16 ? 1 : 2; }

// The 32x32x2 kernel: m > 16 (below that the 16x16x4 kernel, with half the
// padded MFMA work, measured faster) and the alignment its clamped float4 A
// loads need.
bool use_w32(int m, int k, const float* A, int lda) {
  return m > 16 && k >= 4 && k % 4 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
}

// Compute units of the current device: the stream-K grids take one
// workgroup per CU.
int cu_count() { return bch::device_cu_count(); }

// FMA path: k rows per split and split count.
void fma_plan(int k, int* kchunk, int* splits) {
  int s = kFmaSplits;
  if (k < kFmaSplits * 4 * kFmaUnroll) s = (k + 4 * kFmaUnroll - 1) / (4 * kFmaUnroll);
  if (s < 1) s = 1;
  const int kc = (k + s - 1) / s;
  *kchunk = kc;
  *splits = (k + kc - 1) / kc;
}

// Stream-K path: units, workgroups (one per CU; on the staged-A path more
// when a run's A^T slice would not fit in LDS), units per workgroup, and
// partial slots per group.
struct SkPlan {
  long long U = 0;
  int cg = 0, kb = 0, G = 0, upw = 0, smax = 0, mb = 1;
  size_t lds = 0;
};

// A operand per unit in registers: needs whole, aligned float4 rows of A.
bool sk_areg(int k, const float* A, int lda) {
  return k % 4 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
}

SkPlan sk_plan(int m, int n, int k, bool areg) {
  SkPlan p;
  p.mb = sk_mb(m);
  p.cg = (n + kSkCols - 1) / kSkCols;
  p.kb = (k + kSkRows - 1) / kSkRows;
  p.U = (long long)p.cg * p.kb;
  long long g = cu_count();
  if (!areg) {
    const int cap = (kLdsBytes / (4 * 16 * p.mb) - 4) / kSkRows;  // units whose A^T fits in LDS
    if ((p.U + g - 1) / g > cap) g = (p.U + cap - 1) / cap;
  }
  if (g > p.U) g = p.U;
  p.G = (int)g;
  p.upw = (int)((p.U + p.G - 1) / p.G);
  for (int c = 0; c < p.cg; ++c) {
    const int ns = wg_of_unit((long long)c * p.kb + p.kb - 1, p.U, p.G) - wg_of_unit((long long)c * p.kb, p.U, p.G) + 1;
    if (ns > p.smax) p.smax = ns;
  }
  p.lds = areg ? 0 : sizeof(float) * 16 * p.mb * (size_t)(16 * p.upw + 4);
  return p;
}

// 32x32x2 path: 32-row units, one workgroup per CU.
struct W32Plan {
  long long U = 0;
  int cg = 0, nblk = 0, G = 0, smax = 0;
};

W32Plan w32_plan(int n, int k) {
  W32Plan p;
  p.cg = (n + kSkCols - 1) / kSkCols;
  p.nblk = (k + kW32Rows - 1) / kW32Rows;
  p.U = (long long)p.cg * p.nblk;
  long long g = cu_count();
  if (g > p.U) g = p.U;
  p.G = (int)g;
  for (int c = 0; c < p.cg; ++c) {
    const int ns = wg_of_unit((long long)c * p.nblk + p.nblk - 1, p.U, p.G) -
                   wg_of_unit((long long)c * p.nblk, p.U, p.G) + 1;
    if (ns > p.smax) p.smax = ns;
  }
  return p;
}

// transposed-weight path: units of 16 rg_rb(m) rows x 8192 / (16 rg_rb(m)) k, one workgroup per CU
struct NtPlan {
  long long U = 0;
  int rb = 0, ng = 0, nkb = 0, G = 0, smax = 0;
};

NtPlan nt_plan(int m, int n, int k) {
  NtPlan p;
  p.rb = rg_rb(m);
  const int rows = 16 * p.rb, ku = 8192 / rows;
  p.ng = (n + rows - 1) / rows;
  p.nkb = (k + ku - 1) / ku;
  p.U = (long long)p.ng * p.nkb;
  long long g = cu_count();
  if (g > p.U) g = p.U;
  p.G = (int)g;
  for (int c = 0; c < p.ng; ++c) {
    const int ns = wg_of_unit((long long)c * p.nkb + p.nkb - 1, p.U, p.G) - wg_of_unit((long long)c * p.nkb, p.U, p.G) + 1;
    if (ns > p.smax) p.smax = ns;
  }
  return p;
}

// the ring kernel's partial blocks (MB RB sums per lane and wave), 256-byte aligned; its flags follow
size_t nt_partial_bytes(const NtPlan& p, int m) {
  const size_t b = sizeof(float) * (size_t)p.ng * (size_t)p.smax * 4 * (m <= 16 ? 1 : 2) * p.rb * 64;
  return (b + 255) & ~(size_t)255;
}

// one epoch per launch of the ring kernel, process-wide, never 0
std::atomic<unsigned long long> g_nt_epoch{0};

// Whole-row path for transposed weights: m <= 8 and every wave of every CU
// gets at least one row.
int rows_mt(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

bool use_rows(int m, int n, int k) {
  (void)k;
  return m <= 8 && n >= kRowWaves * cu_count();
}

template <int MT>
hipError_t launch_rows(hipStream_t s, int m, int n, int k, const float* A, int lda, const float* W, int ldw, float* C,
                       int ldc, const float* bias, int act) {
  const bool edge = k % kRowPass != 0;
  const void* f = edge ? reinterpret_cast<const void*>(sgemm_skinny_nt_rows<MT, true>)
                       : reinterpret_cast<const void*>(sgemm_skinny_nt_rows<MT, false>);
  hipError_t e = bch::ensure_dynamic_lds(f, kLdsBytes);
  if (e != hipSuccess) return e;
  // one workgroup per CU, more when a block's rows would not fit in LDS
  const int cap = kRowCap(MT);
  const int g = std::max(cu_count(), (n + cap - 1) / cap);
  const int rmax = (n + g - 1) / g;
  const int lds = (int)(sizeof(float) * ((size_t)kRowRed + (size_t)rmax * kRowWaves * MT));
  const dim3 grid(g), block(64 * kRowWaves);
  if (edge)
    hipLaunchKernelGGL((sgemm_skinny_nt_rows<MT, true>), grid, block, lds, s, m, n, k, A, lda, W, ldw, C, ldc, bias,
                       act);
  else
    hipLaunchKernelGGL((sgemm_skinny_nt_rows<MT, false>), grid, block, lds, s, m, n, k, A, lda, W, ldw, C, ldc, bias,
                       act);
  return hipGetLastError();
}

template <bool EDGE, int MB>
hipError_t launch_w32(hipStream_t s, const W32Plan& p, int m, int n, int k, const float* A, int lda, const float* B,
                      int ldb, float* P) {
  hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(sgemm_skinny_w32<kW32PF, EDGE, MB>), kW32Lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((sgemm_skinny_w32<kW32PF, EDGE, MB>), dim3(p.G), dim3(256), kW32Lds, s, m, n, k, A, lda, B,
                     ldb, P, p.U, p.G, p.nblk, p.smax);
  return hipGetLastError();
}

template <int MB, bool AREG>
hipError_t launch_sk(hipStream_t s, const SkPlan& p, int m, int n, int k, const float* A, int lda, const float* B,
                     int ldb, float* P) {
  if (!AREG) {
    hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(sgemm_skinny_sk<MB, AREG>), kLdsBytes);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((sgemm_skinny_sk<MB, AREG>), dim3(p.G), dim3(256), p.lds, s, m, n, k, A, lda, B, ldb, P, p.U,
                     p.G, p.kb, p.smax);
  return hipGetLastError();
}

struct RingArgs {
  float* P;
  unsigned long long* F;
  unsigned long long epoch;
  float* C;
  int ldc;
  const float* bias;
  int act;
};

template <int MB, int RB, bool EDGE>
hipError_t launch_nt_ring(hipStream_t s, const NtPlan& p, int m, int n, int k, const float* A, int lda,
                          const float* W, int ldw, const RingArgs& r) {
  const void* f = reinterpret_cast<const void*>(sgemm_skinny_nt_ring<MB, RB, EDGE>);
  hipError_t e = bch::ensure_dynamic_lds(f, rg_lds_bytes<MB, RB>());
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((sgemm_skinny_nt_ring<MB, RB, EDGE>), dim3(p.G), dim3(512), (rg_lds_bytes<MB, RB>()), s, m, n,
                     k, A, lda, W, ldw, r.C, r.ldc, r.bias, r.act, r.P, r.F, r.epoch, p.U, p.G, p.nkb, p.smax,
                     bch::launch_ctl().fault, bch::launch_ctl().spin);
  return hipGetLastError();
}

}  // namespace

namespace bch {

bool sgemm_skinny_nt_applies(int m, int n, int k, const float* A, int lda, const float* W, int ldw) {
  if (m < 1 || m > 32 || n < 1 || k < 4 || k % 4 != 0 || lda % 4 != 0 || ldw % 4 != 0) return false;
  if (A && (reinterpret_cast<uintptr_t>(A) & 15) != 0) return false;
  if (W && (reinterpret_cast<uintptr_t>(W) & 15) != 0) return false;
  return true;
}

size_t sgemm_skinny_nt_workspace_bytes(int m, int n, int k) {
  if (use_rows(m, n, k)) return 0;
  const NtPlan p = nt_plan(m, n, k);
  return nt_partial_bytes(p, m) + sizeof(unsigned long long) * (size_t)p.ng * (size_t)p.smax * 4;
}

hipError_t launch_sgemm_skinny_nt(hipStream_t s, int m, int n, int k, const float* A, int lda, const float* W,
                                  int ldw, float* C, int ldc, void* ws, size_t ws_bytes, const float* bias,
                                  int act) {
  if (use_rows(m, n, k)) {
    const int mt = rows_mt(m);
    if (mt == 1) return launch_rows<1>(s, m, n, k, A, lda, W, ldw, C, ldc, bias, act);
    if (mt == 2) return launch_rows<2>(s, m, n, k, A, lda, W, ldw, C, ldc, bias, act);
    if (mt == 4) return launch_rows<4>(s, m, n, k, A, lda, W, ldw, C, ldc, bias, act);
    return launch_rows<8>(s, m, n, k, A, lda, W, ldw, C, ldc, bias, act);
  }
  if (ws == nullptr || ws_bytes < sgemm_skinny_nt_workspace_bytes(m, n, k)) return hipErrorInvalidValue;
  const NtPlan p = nt_plan(m, n, k);
  RingArgs r{static_cast<float*>(ws),
             reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + nt_partial_bytes(p, m)),
             ++g_nt_epoch, C, ldc, bias, act};
  if (m <= 16) {  // rg_rb(m) == 2
    const bool edge = k % RgShape<2>::KU != 0;
    return edge ? launch_nt_ring<1, 2, true>(s, p, m, n, k, A, lda, W, ldw, r)
                : launch_nt_ring<1, 2, false>(s, p, m, n, k, A, lda, W, ldw, r);
  }
  const bool edge = k % RgShape<4>::KU != 0;  // rg_rb(m) == 4
  return edge ? launch_nt_ring<2, 4, true>(s, p, m, n, k, A, lda, W, ldw, r)
              : launch_nt_ring<2, 4, false>(s, p, m, n, k, A, lda, W, ldw, r);
}

size_t sgemm_skinny_workspace_bytes(int m, int n, int k) {
  if (use_fma(m)) {
    int kc, s;
    fma_plan(k, &kc, &s);
    return sizeof(float) * (size_t)s * (size_t)m * (size_t)n;
  }
  // the largest of the MFMA paths' needs (which one runs depends on A's alignment)
  size_t bytes = 0;
  for (const bool areg : {false, true}) {
    if (m > 32) break;  // 32 < m <= 64: the 64-row w32 kernel only
    const SkPlan p = sk_plan(m, n, k, areg);
    const size_t b1 = sizeof(float) * (size_t)p.cg * (size_t)p.smax * (size_t)m * kSkCols;
    if (b1 > bytes) bytes = b1;
  }
  if (m > 16) {
    const W32Plan q = w32_plan(n, k);
    const size_t b2 = sizeof(float) * (size_t)q.cg * (size_t)q.smax * (size_t)m * kSkCols;
    if (b2 > bytes) bytes = b2;
  }
  return bytes;
}

bool sgemm_skinny_applies(int m, int n, int k, const float* A, int lda, const float* B, int ldb) {
  if (m < 1 || m > 64 || n < 4 || k < 1) return false;
  if (n % 4 != 0 || ldb % 4 != 0) return false;
  if (m > 32 && !use_w32(m, k, A, lda)) return false;  // 32 < m <= 64: the 64-row w32 kernel only
  if (B && (reinterpret_cast<uintptr_t>(B) & 15) != 0) return false;
  return true;
}

const char* sgemm_skinny_kernel_name(int m) {
  if (use_fma(m)) return "sgemm_skinny_fma";
  if (m > 32) return "sgemm_skinny_w32<2>";  // two 32-row blocks per unit
  if (m > 16) return "sgemm_skinny_w32";  // with K % 4 == 0 and aligned A, as at the configs
  return sk_mb(m) == 1 ? "sgemm_skinny_sk<1>" : "sgemm_skinny_sk<2>";
}

hipError_t launch_sgemm_skinny(hipStream_t s, int m, int n, int k, const float* A, int lda,
                               const float* B, int ldb, float* C, int ldc, void* ws, size_t ws_bytes,
                               const float* bias, int act) {
  if (ws == nullptr || ws_bytes < sgemm_skinny_workspace_bytes(m, n, k)) return hipErrorInvalidValue;
  float* P = static_cast<float*>(ws);
  const dim3 rgrid((unsigned)((n + 255) / 256), (unsigned)m);
  if (use_fma(m)) {
    int kchunk, splits;
    fma_plan(k, &kchunk, &splits);
    dim3 grid((n + kFmaCols - 1) / kFmaCols, splits), block(256);
    if (m == 1)
      hipLaunchKernelGGL(sgemm_skinny_fma<1>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
    else if (m == 2)
      hipLaunchKernelGGL(sgemm_skinny_fma<2>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
    else
      hipLaunchKernelGGL(sgemm_skinny_fma<4>, grid, block, 0, s, m, n, k, A, lda, B, ldb, P, kchunk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sgemm_skinny_reduce, rgrid, dim3(256), 0, s, m, n, P, splits, C, ldc, bias, act);
    return hipGetLastError();
  }
  if (use_w32(m, k, A, lda)) {
    const W32Plan q = w32_plan(n, k);
    hipError_t e = m > 32 ? (k % kW32Rows == 0 ? launch_w32<false, 2>(s, q, m, n, k, A, lda, B, ldb, P)
                                               : launch_w32<true, 2>(s, q, m, n, k, A, lda, B, ldb, P))
                          : (k % kW32Rows == 0 ? launch_w32<false, 1>(s, q, m, n, k, A, lda, B, ldb, P)
                                               : launch_w32<true, 1>(s, q, m, n, k, A, lda, B, ldb, P));
    if (e != hipSuccess) return e;
    return launch_sk_reduce(s, m, n, P, q.U, q.G, q.nblk, q.smax, C, ldc, bias, act, kSkCols);
  }
  const bool areg = sk_mb(m) == 1 && sk_areg(k, A, lda);
  const SkPlan p = sk_plan(m, n, k, areg);
  hipError_t e;
  if (p.mb == 1)
    e = areg ? launch_sk<1, true>(s, p, m, n, k, A, lda, B, ldb, P) : launch_sk<1, false>(s, p, m, n, k, A, lda, B, ldb, P);
  else  // m > 16 with aligned A takes the 32x32x2 kernel above
    e = launch_sk<2, false>(s, p, m, n, k, A, lda, B, ldb, P);
  if (e != hipSuccess) return e;
  return launch_sk_reduce(s, m, n, P, p.U, p.G, p.kb, p.smax, C, ldc, bias, act, kSkCols);
}

}  // namespace bch
