// dgemm_mfma.hip -- f64 GEMM on the gfx950 FP64 matrix cores.
//
// Replaces GemmF64::{execute, execute_gemm, execute_gemm_ex} and
// GemmCachedF64 (crates/barracuda/src/ops/linalg/gemm_f64.rs:77-456;
// shaders/linalg/gemm_f64.wgsl, a 16x16 scalar tile).  Contract, batched:
//   C[b] = alpha op(A[b]) op(B[b]) (+ beta C[b] when beta != 0),
// op(A) = A ([m][k]) or A^T (A stored [k][m]), op(B) = B ([k][n]) or B^T
// (B stored [n][k]), f64 throughout.  With beta == 0, C is not read (the
// shader's `if (params.beta != 0.0)`, gemm_f64.wgsl:84-89).
//
// Design:
//   * v_mfma_f64_16x16x4_f64: a wavefront multiplies a 16x4 A block by a
//     4x16 B block into a 16x16 f64 accumulator (4 values per lane).  Lane l
//     supplies A[l%16][l/16] and B[l/16][l%16]; value r of lane l is
//     C[l/16 + 4*r][l%16] (rows interleave across the lane quarters, unlike
//     the f32 16x16 MFMAs' 4*(l/16) + r; checked by the 2 x 2 and ragged
//     GEMM tests, which a row permutation fails).  The k index a lane quarter feeds is free, so
//     quarter q takes k = 4q + s in step s of a 16-wide k-tile: four
//     consecutive k per lane, two 128-bit LDS reads per operand block.
//   * Block tile 128 x 128 x 16, four wavefronts in a 2x2 grid, each owning
//     64 x 64 as 4 x 4 MFMA blocks (128 accumulator registers).  LDS holds
//     both tiles k-contiguous ([m][k], [n][k]), rows padded to 18 doubles so
//     the 16 rows a read phase touches fall in distinct banks; double
//     buffered (2 x 36 KB), so two workgroups fit on a CU.
//   * Tile loads: an operand whose rows are k-contiguous (A, or B^T stored
//     [n][k]) is copied row by row (8 lanes x 16 bytes per 128-byte row);
//     one whose rows run along m or n (B [k][n], or A^T stored [k][m]) is
//     loaded as 2 x 2 blocks and written transposed, the 8 lanes of a store
//     phase covering one LDS row (no bank conflicts) -- except on the
//     unguarded path, where B [k][n] (and A^T beside it) stays [k][rows] in
//     LDS and a fragment's two k are read as one ds_read2_b64.  The
//     transpose through registers left the staged registers permuted across
//     the loop's back edge, and every iteration ended copying them into
//     place behind a wait for all of the next tile's loads.  4096^3 NN
//     72.5-72.9 -> 73.9-74.0 TFLOP/s, TN 71.2-71.5 -> 74.1-74.2, 2048^3
//     69.0 -> 71.2 (one box, two runs each); A^T kept [k][m] with B^T given
//     [n][k] (TT), 72.6-72.7 -> 73.6-73.9 (one 4-byte spill, outside the
//     loop).
//   * Software pipeline: a k-tile's fragments are read in two halves, the
//     second half of tile t under the MFMAs of its first two steps and the
//     first half of tile t + 1 (after the one barrier per tile) under its
//     last two; global loads run two tiles ahead of the MFMAs.  Measured at
//     4096^3 against loading one tile ahead and reading all fragments at the
//     top of the tile: 59.7 -> 63.4 TFLOP/s.
//   * The LDS stores and global loads of a tile are spread between the
//     MFMAs of the first half (one of each per two MFMAs) rather than issued
//     as a burst at the top of the tile, where the four wavefronts of a
//     workgroup arrive together from the barrier: 4096^3 67.6 -> 72.5
//     TFLOP/s (86.0% -> 92.2%).  A register-only loop of independent
//     v_mfma_f64_16x16x4_f64 sustains 99% of the FP64 matrix peak from one
//     wavefront per SIMD, so what remains is the barrier and memory issue.
//   * Workgroup -> tile mapping is XCD-aware and grouped, as in the f32 GEMM.
//   * Split k: when the output has fewer 128 x 128 tiles than the device has
//     CUs (a skinny m or n, e.g. the P V product of an attention), the k
//     range is cut into nsplit contiguous runs of whole 16-wide k-tiles
//     (at least 8 k-tiles each); grid.y = batch x nsplit.  Each workgroup
//     writes its raw accumulators to a partial [batch][nsplit][m][n] in the
//     context's workspace, and dgemm_split_reduce adds the nsplit partials of
//     each element in split order (deterministic), then applies alpha and
//     beta C.
//   * CHECK=false needs m % 128 == 0, n % 128 == 0, k % 16 == 0, even
//     leading dimensions and batch strides, 16-byte aligned A and B; CHECK
//     guards every load (zero fill) and store.  With CHECK, V2 guards each
//     pair of doubles as one range-checked 128-bit buffer load where pairs
//     cannot straddle an operand's edge (the paired dimension even, even
//     leading dimensions and strides, aligned bases); scalar guards serve
//     the rest.  Against scalar guards (two conditional 8-byte loads per
//     pair): 4000^3 55.0 -> 68.5 TFLOP/s, 4000^3 with both operands
//     transposed 50.5 -> 68.6, 3000 x 5000 x 1000 49.6 -> 62.6.
#include "bch_internal.h"

#include <stdint.h>

#include <algorithm>

namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

constexpr int kDT = 256;  // threads
constexpr int kDBK = 16;
constexpr int kDLDK = kDBK + 2;  // padded LDS row, doubles

struct d2 {
  double x, y;
};

__device__ __forceinline__ d2 ld2(const double* p) { return *reinterpret_cast<const d2*>(p); }

constexpr unsigned kBad = 0x80000000u;  // a byte offset past every operand's buffer resource

__device__ __forceinline__ d2 ld2_rs(__amdgpu_buffer_rsrc_t rs, unsigned off) {
  return __builtin_bit_cast(d2, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// Global -> registers for one ROWS-row x 16-k operand tile of op(X).
// KCONT: row r, element k of op(X) is X[r * ld + k] (rows k-contiguous);
// otherwise it is X[k * ld + r] (the stored matrix is [k][rows]).
// Registers: ROWS / 32 pairs of doubles per thread either way.
// CHECK guards each element (zero outside rows x K).  CHECK && V2 loads each
// pair with one range-checked 128-bit buffer load from `rs`: the host takes
// this form only when a pair lies wholly inside or wholly outside the
// operand (the paired dimension even, ld and strides even, 16-byte aligned
// bases) and the operand spans less than 2^31 bytes; outside, the offset is
// kBad and the hardware returns zeros.
template <int ROWS, bool KCONT, bool CHECK, bool V2>
__device__ __forceinline__ void load_dtile(const double* __restrict__ X, __amdgpu_buffer_rsrc_t rs, int ld, int rows,
                                           int K, int r0, int k0, int tid, d2 (&reg)[ROWS / 32]) {
  if (KCONT) {
    // pair f: row tid / 8 + 32 f, k 2 * (tid % 8)
#pragma unroll
    for (int f = 0; f < ROWS / 32; ++f) {
      const int r = r0 + tid / 8 + 32 * f, k = k0 + 2 * (tid % 8);
      if (!CHECK) {
        reg[f] = ld2(X + (long long)r * ld + k);
      } else if (V2) {
        reg[f] = ld2_rs(rs, (r < rows && k < K) ? ((unsigned)r * (unsigned)ld + (unsigned)k) * 8u : kBad);
      } else {
        reg[f].x = (r < rows && k < K) ? X[(long long)r * ld + k] : 0.0;
        reg[f].y = (r < rows && k + 1 < K) ? X[(long long)r * ld + k + 1] : 0.0;
      }
    }
  } else {
    // 2 x 2 block q (q < ROWS / 64): blk = tid + 256 q, kq = blk % 8, rq = blk / 8;
    // reg[2q + e] = X[k0 + 2 kq + e][r0 + 2 rq .. +1]
#pragma unroll
    for (int q = 0; q < ROWS / 64; ++q) {
      const int blk = tid + kDT * q, kq = blk % 8, rq = blk / 8;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int k = k0 + 2 * kq + e, r = r0 + 2 * rq;
        if (!CHECK) {
          reg[2 * q + e] = ld2(X + (long long)k * ld + r);
        } else if (V2) {
          reg[2 * q + e] =
              ld2_rs(rs, (k < K && r < rows) ? ((unsigned)k * (unsigned)ld + (unsigned)r) * 8u : kBad);
        } else {
          reg[2 * q + e].x = (k < K && r < rows) ? X[(long long)k * ld + r] : 0.0;
          reg[2 * q + e].y = (k < K && r + 1 < rows) ? X[(long long)k * ld + r + 1] : 0.0;
        }
      }
    }
  }
}

// registers -> LDS tile [ROWS][kDLDK] (k-contiguous)
template <int ROWS, bool KCONT>
__device__ __forceinline__ void store_dtile(double* __restrict__ s, int tid, const d2 (&reg)[ROWS / 32]) {
  if (KCONT) {
#pragma unroll
    for (int f = 0; f < ROWS / 32; ++f) {
      const int r = tid / 8 + 32 * f, k = 2 * (tid % 8);
      *reinterpret_cast<d2*>(s + r * kDLDK + k) = reg[f];
    }
  } else {
#pragma unroll
    for (int q = 0; q < ROWS / 64; ++q) {
      const int blk = tid + kDT * q, kq = blk % 8, rq = blk / 8;
      // reg[2q + e] holds (k = 2kq + e; rows 2rq, 2rq + 1): row 2rq + c gets (k, k + 1)
      *reinterpret_cast<d2*>(s + (2 * rq) * kDLDK + 2 * kq) = d2{reg[2 * q].x, reg[2 * q + 1].x};
      *reinterpret_cast<d2*>(s + (2 * rq + 1) * kDLDK + 2 * kq) = d2{reg[2 * q].y, reg[2 * q + 1].y};
    }
  }
}

// An unguarded operand stored [k][rows] (B as [k][n], or A^T as [k][m]) is kept the same
// way in LDS, [16][ROWS + 2] doubles: rows of the tile copied with 128-bit loads and stores,
// ROWS / 2 threads per k row.  Its fragments are then read as two 64-bit values (k and k + 1)
// instead of one 128-bit read of a transposed tile.
template <int ROWS>
__device__ __forceinline__ void load_krow(const double* __restrict__ X, int ld, int r0, int k0, int tid,
                                          d2 (&reg)[ROWS / 32]) {
  constexpr int TPR = ROWS / 2, RSTEP = kDT / TPR;
  const int kr = tid / TPR, c = 2 * (tid % TPR);
  const double* base = X + (long long)(k0 + kr) * ld + r0 + c;
  const long long step = (long long)RSTEP * ld;  // wave-uniform
#pragma unroll
  for (int f = 0; f < ROWS / 32; ++f) reg[f] = ld2(base + f * step);
}

template <int ROWS>
__device__ __forceinline__ void store_krow(double* __restrict__ s, int tid, const d2 (&reg)[ROWS / 32]) {
  constexpr int TPR = ROWS / 2, RSTEP = kDT / TPR;
  const int kr = tid / TPR, c = 2 * (tid % TPR);
#pragma unroll
  for (int f = 0; f < ROWS / 32; ++f) *reinterpret_cast<d2*>(s + (kr + f * RSTEP) * (ROWS + 2) + c) = reg[f];
}

// BM x BN block tile (2 x 2 waves of (BM/2) x (BN/2), TM x TN MFMA blocks each);
// OCC workgroups per CU.
// grid.y = batch * nsplit; with nsplit > 1 the workgroup covers k in
// [split * ksplit, min(K, (split + 1) * ksplit)) and writes its raw sums to
// P (dense [batch][nsplit][M][N]); alpha, beta and C are then unused.
template <int BM, int BN, int OCC, bool TA, bool TB, bool CHECK, bool V2>
__global__ __launch_bounds__(kDT, OCC) void dgemm_mfma_kernel(
    int M, int N, int K, double alpha, const double* __restrict__ A, int lda, long long sA,
    const double* __restrict__ B, int ldb, long long sB, double beta, double* __restrict__ C, int ldc,
    long long sC, int tiles_m, int tiles_n, int nsplit, int ksplit, double* __restrict__ P) {
  constexpr int kDBM = BM, kDBN = BN, TM = BM / 32, TN = BN / 32;
  __shared__ double As[2][kDBM * kDLDK];
  __shared__ double Bs[2][kDBN * kDLDK];

  // ---- tile mapping (XCD-aware, grouped; as sgemm_mfma_kernel) ----
  const int ntiles = tiles_m * tiles_n;
  const int p = blockIdx.x;
  int lt = p;
  if ((ntiles & 7) == 0) lt = (p & 7) * (ntiles >> 3) + (p >> 3);
  constexpr int GROUP = 8;
  const int group_size = GROUP * tiles_n;
  const int g = lt / group_size;
  const int first_m = g * GROUP;
  const int gm = min(tiles_m - first_m, GROUP);
  const int within = lt - g * group_size;
  const int m0 = (first_m + within % gm) * kDBM, n0 = (within / gm) * kDBN;

  const long long bz = blockIdx.y / nsplit;
  const int split = blockIdx.y - (int)bz * nsplit;
  const int kbeg = split * ksplit, kend = (int)min((long long)K, (long long)kbeg + ksplit);
  A += bz * sA;
  B += bz * sB;
  C += bz * sC;
  // buffer resources over this batch's operands (used by CHECK && V2 only)
  const int a_bytes = (int)((TA ? (long long)(K - 1) * lda + M : (long long)(M - 1) * lda + K) * 8);
  const int b_bytes = (int)((TB ? (long long)(N - 1) * ldb + K : (long long)(K - 1) * ldb + N) * 8);
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(A), 0, a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(B), 0, b_bytes, 0x00020000);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lq = lane >> 4;
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);

  d2 ra[BM / 32], rb[BN / 32];
  f64x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (f64x4){0.0, 0.0, 0.0, 0.0};

  // Pipeline: fragments of a k-tile come in two halves (k 4lq .. +1 feed
  // steps 0, 1; k 4lq + 2 .. +3 feed steps 2, 3).  Iteration t stores tile
  // t + 1 (loaded during iteration t - 1) into the buffer the previous
  // barrier released and issues the loads of tile t + 2; phase 0 reads the
  // second halves of tile t under the MFMAs of steps 0, 1; after the one
  // barrier, phase 1 reads the first halves of tile t + 1 under the MFMAs of
  // steps 2, 3.  Tile indices past the end are clamped to the last tile
  // (reloaded, never used).  Scheduling groups pin the interleave.
  const int nk = (kend - kbeg + kDBK - 1) / kDBK;
  const int lastk = kbeg + (nk - 1) * kDBK;
  d2 a[TM][2], b[TN][2];
  constexpr bool AROW = TA && !CHECK, BROW = !TB && !CHECK;
  static_assert(16 * (BM + 2) <= BM * kDLDK && 16 * (BN + 2) <= BN * kDLDK, "k-row tiles fit the buffers");
  auto read_half = [&](int buf, int h) {
    if constexpr (AROW) {
      const double* as = As[buf] + (4 * lq + 2 * h) * (BM + 2) + wm + li;
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i][h] = d2{as[16 * i], as[BM + 2 + 16 * i]};
    } else {
      const double* as = As[buf] + (wm + li) * kDLDK + 4 * lq + 2 * h;
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i][h] = *reinterpret_cast<const d2*>(as + i * 16 * kDLDK);
    }
    if constexpr (BROW) {
      const double* bs = Bs[buf] + (4 * lq + 2 * h) * (BN + 2) + wn + li;
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j][h] = d2{bs[16 * j], bs[BN + 2 + 16 * j]};
    } else {
      const double* bs = Bs[buf] + (wn + li) * kDLDK + 4 * lq + 2 * h;
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j][h] = *reinterpret_cast<const d2*>(bs + j * 16 * kDLDK);
    }
  };
  auto load_tiles = [&](int k0) {
    if constexpr (AROW) load_krow<BM>(A, lda, m0, k0, tid, ra);
    else load_dtile<BM, !TA, CHECK, V2>(A, rsa, lda, M, kend, m0, k0, tid, ra);
    if constexpr (BROW) load_krow<BN>(B, ldb, n0, k0, tid, rb);
    else load_dtile<BN, TB, CHECK, V2>(B, rsb, ldb, N, kend, n0, k0, tid, rb);
  };
  auto store_tiles = [&](int buf) {
    if constexpr (AROW) store_krow<BM>(As[buf], tid, ra);
    else store_dtile<BM, !TA>(As[buf], tid, ra);
    if constexpr (BROW) store_krow<BN>(Bs[buf], tid, rb);
    else store_dtile<BN, TB>(Bs[buf], tid, rb);
  };
  auto mfma_half = [&](int h) {
    // step s = 2h + e uses k = 4 lq + s
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const double av = e ? a[i][h].y : a[i][h].x;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const double bv = e ? b[j][h].y : b[j][h].x;
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc[i][j], 0, 0, 0);
        }
      }
  };
  // LDS reads per half: one per block either way (a k-row operand's two 64-bit values, 130 or
  // more doubles apart, are one ds_read2_b64)
  constexpr int NR = TM + TN;
  constexpr int NM = 2 * TM * TN;                                 // MFMAs per half
  static_assert(NM >= 2 * NR, "half tile too small to cover its reads");

  if (nk > 0) {
    if constexpr (AROW || BROW) {
      load_tiles(kbeg);
      store_tiles(0);
      load_tiles(min(kbeg + kDBK, lastk));
    } else {
      load_dtile<BM, !TA, CHECK, V2>(A, rsa, lda, M, kend, m0, kbeg, tid, ra);
      load_dtile<BN, TB, CHECK, V2>(B, rsb, ldb, N, kend, n0, kbeg, tid, rb);
      store_dtile<BM, !TA>(As[0], tid, ra);
      store_dtile<BN, TB>(Bs[0], tid, rb);
      load_dtile<BM, !TA, CHECK, V2>(A, rsa, lda, M, kend, m0, min(kbeg + kDBK, lastk), tid, ra);
      load_dtile<BN, TB, CHECK, V2>(B, rsb, ldb, N, kend, n0, min(kbeg + kDBK, lastk), tid, rb);
    }
  }
  __syncthreads();
  if (nk > 0) read_half(0, 0);

  constexpr int NW = BM / 32 + BN / 32;  // LDS stores (= 128-bit global loads) per thread per tile
  constexpr int RM = NM >= 2 * NR + 2 * NW ? 2 : 1;  // MFMAs after each read in phase 0
  static_assert(NM >= RM * NR + 2 * NW, "half tile too small to cover its reads, stores and loads");
  for (int t = 0; t < nk; ++t) {
    const int cur = t & 1;
    read_half(cur, 1);
    if constexpr (AROW || BROW) {
      store_tiles(cur ^ 1);
      load_tiles(min(kbeg + (t + 2) * kDBK, lastk));
    } else {
      store_dtile<BM, !TA>(As[cur ^ 1], tid, ra);
      store_dtile<BN, TB>(Bs[cur ^ 1], tid, rb);
      load_dtile<BM, !TA, CHECK, V2>(A, rsa, lda, M, kend, m0, min(kbeg + (t + 2) * kDBK, lastk), tid, ra);
      load_dtile<BN, TB, CHECK, V2>(B, rsb, ldb, N, kend, n0, min(kbeg + (t + 2) * kDBK, lastk), tid, rb);
    }
    mfma_half(0);
    // Phase 0 order: the second-half reads of tile t, one per 2 MFMAs, then
    // the LDS stores of tile t + 1 and the global loads of tile t + 2, a
    // store and a load per 2 MFMAs, so no burst of memory instructions
    // holds up a wavefront's MFMAs.
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, RM, 0);
    }
#pragma unroll
    for (int r = 0; r < NW; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    if (NM > RM * NR + 2 * NW) __builtin_amdgcn_sched_group_barrier(0x008, NM - RM * NR - 2 * NW, 0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_half(cur ^ 1, 0);
    mfma_half(1);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM - 2 * NR, 0);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- epilogue: value r of lane (lq, li) is row lq + 4 r, col li of the block ----
  if (nsplit > 1) {
    double* part = P + (bz * nsplit + split) * (long long)M * N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn + 16 * j + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm + 16 * i + lq + 4 * r;
          if (!CHECK || (row < M && col < N)) part[(long long)row * N + col] = acc[i][j][r];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn + 16 * j + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm + 16 * i + lq + 4 * r;
        if (!CHECK || (row < M && col < N)) {
          double* c = C + (long long)row * ldc + col;
          const double v = alpha * acc[i][j][r];
          *c = beta != 0.0 ? v + beta * *c : v;
        }
      }
    }
  }
}

// C[b][row][col] = alpha * sum_{s < nsplit} P[b][s][row][col] (+ beta C when
// beta != 0), the partials added in split order; one element per thread.
__global__ __launch_bounds__(256) void dgemm_split_reduce(int M, int N, int nsplit, const double* __restrict__ P,
                                                          double alpha, double beta, double* __restrict__ C, int ldc,
                                                          long long sC, long long total) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const long long mn = (long long)M * N;
  const long long b = e / mn, rc = e - b * mn;
  const int row = (int)(rc / N), col = (int)(rc - (long long)row * N);
  const double* p = P + b * nsplit * mn + rc;
  double sum = 0.0;
  for (int s = 0; s < nsplit; ++s) sum += p[s * mn];
  double* c = C + b * sC + (long long)row * ldc + col;
  const double v = alpha * sum;
  *c = beta != 0.0 ? v + beta * *c : v;
}

struct SplitPlan {
  int nsplit, ksplit;
};

// Split k only when the output has fewer tiles than the device has CUs, into
// runs of at least 8 k-tiles, and never past grid.y's 65535.
SplitPlan split_plan(int batch, int m, int n, int k, int BM, int BN) {
  const long long tiles = (long long)((m + BM - 1) / BM) * ((n + BN - 1) / BN) * batch;
  const int nk = (k + kDBK - 1) / kDBK;
  const long long cus = bch::device_cu_count();
  long long want = tiles >= cus ? 1 : (cus + tiles - 1) / tiles;
  want = std::min<long long>(want, nk / 8);
  want = std::min<long long>(want, 65535 / std::max(batch, 1));
  if (want <= 1) return {1, nk * kDBK};
  const int per = (int)((nk + want - 1) / want);  // k-tiles per split
  return {(nk + per - 1) / per, per * kDBK};
}

template <int BM, int BN, int OCC, bool TA, bool TB, bool CHECK, bool V2>
hipError_t launch_d(hipStream_t s, int batch, int m, int n, int k, double alpha, const double* A, int lda,
                    long long sA, const double* B, int ldb, long long sB, double beta, double* C, int ldc,
                    long long sC, void* ws, size_t ws_bytes) {
  const int tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if ((long long)tm * tn > 0x7fffffffLL || batch > 65535) return hipErrorInvalidValue;
  const SplitPlan sp = split_plan(batch, m, n, k, BM, BN);
  const long long total = (long long)batch * m * n;
  if (sp.nsplit > 1 && (!ws || ws_bytes < (size_t)total * sp.nsplit * sizeof(double))) return hipErrorInvalidValue;
  double* P = sp.nsplit > 1 ? static_cast<double*>(ws) : nullptr;
  hipLaunchKernelGGL((dgemm_mfma_kernel<BM, BN, OCC, TA, TB, CHECK, V2>), dim3(tm * tn, batch * sp.nsplit), dim3(kDT), 0,
                     s, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, tm, tn, sp.nsplit,
                     sp.nsplit > 1 ? sp.ksplit : (k > 0 ? k : 1), P);
  if (sp.nsplit > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(dgemm_split_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, m, n, sp.nsplit,
                       P, alpha, beta, C, ldc, sC, total);
  }
  return hipGetLastError();
}

#ifndef BCH_DGEMM_TILE_M  // tile choice (a build-time knob for tuning sweeps)
#define BCH_DGEMM_TILE_M 128
#define BCH_DGEMM_TILE_N 128
#define BCH_DGEMM_OCC 2
#endif
constexpr int kDTileM = BCH_DGEMM_TILE_M, kDTileN = BCH_DGEMM_TILE_N, kDOcc = BCH_DGEMM_OCC;

template <bool TA, bool TB>
hipError_t launch_ab(hipStream_t s, int batch, int m, int n, int k, double alpha, const double* A, int lda,
                     long long sA, const double* B, int ldb, long long sB, double beta, double* C, int ldc,
                     long long sC, void* ws, size_t ws_bytes) {
  constexpr int BM = kDTileM, BN = kDTileN, OCC = kDOcc;
  const bool fast = m % BM == 0 && n % BN == 0 && k % kDBK == 0 && lda % 2 == 0 && ldb % 2 == 0 &&
                    sA % 2 == 0 && sB % 2 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(B) & 15) == 0;
  if (fast)
    return launch_d<BM, BN, OCC, TA, TB, false, false>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C,
                                                       ldc, sC, ws, ws_bytes);
  // Pairs of doubles wholly inside or outside each operand: the paired
  // dimension (k for a k-contiguous operand, else its rows) even, leading
  // dimensions and strides even, 16-byte aligned bases; and byte offsets
  // below 2^31.
  const long long a_bytes = (TA ? (long long)(k - 1) * lda + m : (long long)(m - 1) * lda + k) * 8;
  const long long b_bytes = (TB ? (long long)(n - 1) * ldb + k : (long long)(k - 1) * ldb + n) * 8;
  const bool v2 = k > 0 && (TA ? m : k) % 2 == 0 && (TB ? k : n) % 2 == 0 && lda % 2 == 0 && ldb % 2 == 0 &&
                  sA % 2 == 0 && sB % 2 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(B) & 15) == 0 && a_bytes < 0x7fffffffLL && b_bytes < 0x7fffffffLL;
  if (v2)
    return launch_d<BM, BN, OCC, TA, TB, true, true>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc,
                                                     sC, ws, ws_bytes);
  return launch_d<BM, BN, OCC, TA, TB, true, false>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc,
                                                    sC, ws, ws_bytes);
}

}  // namespace

namespace bch {

size_t dgemm_workspace_bytes(int batch, int m, int n, int k) {
  if (batch <= 0 || m <= 0 || n <= 0) return 0;
  const SplitPlan sp = split_plan(batch, m, n, k, kDTileM, kDTileN);
  return sp.nsplit > 1 ? (size_t)batch * m * n * sp.nsplit * sizeof(double) : 0;
}

int dgemm_split_count(int batch, int m, int n, int k) {
  if (batch <= 0 || m <= 0 || n <= 0) return 1;
  return split_plan(batch, m, n, k, kDTileM, kDTileN).nsplit;
}

hipError_t launch_dgemm(hipStream_t s, bool transa, bool transb, int batch, int m, int n, int k, double alpha,
                        const double* A, int lda, long long sA, const double* B, int ldb, long long sB,
                        double beta, double* C, int ldc, long long sC, void* ws, size_t ws_bytes) {
  if (batch <= 0 || m <= 0 || n <= 0) return hipSuccess;
  if (transa) {
    if (transb)
      return launch_ab<true, true>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, ws, ws_bytes);
    return launch_ab<true, false>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, ws, ws_bytes);
  }
  if (transb)
    return launch_ab<false, true>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, ws, ws_bytes);
  return launch_ab<false, false>(s, batch, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, ws, ws_bytes);
}

}  // namespace bch
