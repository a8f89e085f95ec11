// sgemm_mfma.hip -- f32 GEMM on the gfx950 FP32 matrix cores.
//
// Replaces MatMul::execute (crates/barracuda/src/ops/matmul.rs:89-214; WGSL
// kernels K1 shaders/math/matmul_gpu_evolved_f64.wgsl, K2
// matmul_cpu_tiled_f64.wgsl, K3 matmul_tiled_f64.wgsl), MatmulTiled
// (ops/matmul_tiled.rs:62-122) and BatchMatMul (ops/batch_matmul.rs:47-144,
// K5 batch_matmul_f64.wgsl).  Contract: C[m,n] = sum_p A[m,p] B[p,n], f32
// inputs, f32 accumulation, row-major.
//
// Design:
//   * v_mfma_f32_32x32x2_f32: a wavefront multiplies a 32x2 A block by a 2x32
//     B block into a 32x32 f32 accumulator (16 values per lane).  Lane l
//     supplies A[l%32][l/32] and B[l/32][l%32]; result value r of lane l is
//     C[8*(r/4) + 4*(l/32) + r%4][l%32].
//   * The k index each lane half feeds is free (the MFMA sums over it), so
//     lane half h takes k = 8c + 4h + s in MFMA step s of 8-wide chunk c.
//     Both operands are then 4 consecutive k values per lane: one
//     ds_read_b128 per 32-row block feeds four MFMAs.  To make that true for
//     B as well, B tiles are stored k-contiguous ([n][k]) in LDS: each thread
//     loads a 4(k) x 4(n) block with four 128-bit global loads and writes it
//     transposed with four 128-bit LDS stores, the lanes of a store phase
//     covering one LDS row.  The unguarded 256-row tiles instead keep B
//     row-major in LDS and read each lane's four k as four 32-bit values
//     (BROW in the kernel).
//   * Block tile BM x BN x BK (256x256, 256x128 or 128x128 by shape, see
//     pick_tile), four wavefronts in a 2x2 grid, each owning a (BM/2) x (BN/2)
//     sub-tile of (BM/64) x (BN/64) MFMA blocks (the 256x256 tile with the
//     bias and activation epilogue: eight wavefronts, 2 x 4).  LDS rows
//     are padded by 4 floats so the 128-bit reads of 32 consecutive rows do
//     not collide on banks.  LDS is double-buffered, with one register set
//     staging the global loads: tile t + 1 goes from registers to the other
//     LDS buffer in chunk NC - 2 of tile t, and the loads of tile t + 2 are
//     issued right behind those stores, so every load has a whole tile of
//     MFMAs (and the barrier) to land; one barrier per k-tile.  Measured at
//     4096^3 against issuing tile t + 1's loads at the top of tile t (two
//     chunks to land): 136.8 -> 143.1 TFLOP/s (NN), 141.6 -> 148.1 (B as
//     [n][k], bias + ReLU), 131.6 -> 137.6 (16 x 1024^3 batched).  Two
//     register sets (loads two tiles ahead) spill 274 VGPRs.
//   * Software pipeline inside a tile: the operand fragments are
//     double-buffered by 8-wide chunk, so the LDS reads of chunk c + 1 issue
//     between the MFMAs of chunk c, the next tile's LDS stores issue between
//     the MFMAs of the second-to-last chunk, and the barrier sits before the
//     last chunk's MFMAs (whose fragments are already in registers) while
//     the next tile's first reads overlap them.  Scheduling groups pin that
//     order.  Measured at 4096^3 against the same tiles with each chunk's
//     reads after the previous chunk's MFMAs and the stores, a full LDS wait
//     and the barrier after all of them: 133.0 -> 138.6 TFLOP/s (NN), 135.2
//     -> 142.2 (B as [n][k]), 124 -> 129 (16 x 1024^3 batched).
//   * Workgroup -> tile mapping is XCD-aware: gfx950 dispatches workgroups
//     round-robin over 8 XCDs, so consecutive workgroup ids are remapped to
//     one XCD's contiguous range of tiles, then walked in groups of 8 tile
//     rows so concurrently running tiles share A and B panels in that
//     XCD's L2.  A batched launch gives each XCD a contiguous run of
//     (batch, tile) slots, i.e. whole batches where they divide the run.
//   * CHECK=false needs m % BM == 0, n % BN == 0, k % BK == 0, lda/ldb/
//     strides multiples of 4 and 16-byte aligned A/B; CHECK=true guards
//     every load (zero fill) and store and handles any shape and alignment.
//   * TB: B is given as [n][k] (ldb >= k), C = A B^T -- the linear layer's
//     y = x W^T with W [out, in] (shaders/misc/linear_f64.wgsl, the layers of
//     nn/fused_mlp.rs:38-168).  Its tile is already k-contiguous, so it is
//     loaded like the A tile (128-bit rows straight into LDS [n][k]).
//   * Epilogue: C = act(acc (+ bias[col])) with act none, ReLU or GELU (tanh
//     form), fused into the store -- linear_f64.wgsl adds the bias after the
//     dot product, and fused_mlp runs relu_f64.wgsl (gelu_f64.wgsl for a GELU
//     layer) as a separate pass over the output.  EPI is a
//     template flag so the plain GEMM stores straight from the accumulators
//     (420 VGPRs, no spill at 256x256); the bias/activation variant of that tile
//     parks 8 accumulators in scratch for the epilogue only (36 bytes per
//     lane, no AGPR copies in the k-loop; measured at the plain kernel's
//     rate).
#include "bch_internal.h"

#include <stdint.h>

#include <algorithm>
#include <string>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));


// W8: eight wavefronts (2 x 4, each (BM/2) x (BN/4)) instead of four, two per SIMD.  Taken by the
// 256x256 tile with the bias and activation epilogue, where a SIMD's second wavefront overlaps
// the epilogue's VALU work.  Same box, two runs each (us, 4 -> 8 wavefronts, [out, in] weights
// with bias): GELU 4096^3 951.6 -> 940.0-940.5, 8192 x 4096 x 4096 1895-1897 -> 1873-1874,
// 4096 x 11008 x 4096 2630-2631 -> 2603-2607, 6144^3 3164-3165 -> 3144-3145, 4000^3 (float4
// guards) 941-942 -> 917-918; ReLU 4000^3 922-924 -> 904-905, the others within 0.3%.  Without
// an epilogue the 256x256 tile stays on four wavefronts: eight took 4096^3 146.5 -> 144.8
// TFLOP/s.
template <int BM, int BN, int BK, bool W8 = false>
struct Cfg {
  static constexpr int NT = W8 ? 512 : 256;          // threads per workgroup
  static constexpr int WN = NT / 128;                // waves along n (2 or 4)
  static constexpr int LDK = BK + 4;                 // padded LDS row (floats)
  static constexpr int A_F4 = BM * BK / 4 / NT;  // float4 of A per thread
  static constexpr int B_BLK = BK * BN / 16 / NT;  // 4x4 B blocks per thread
  static constexpr int TM = BM / 64;                 // MFMA blocks per wave (m)
  static constexpr int TN = BN / 32 / WN;            // MFMA blocks per wave (n)
  static constexpr int LDS_FLOATS = 2 * (BM + BN) * LDK;
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");
  static_assert(A_F4 * NT * 4 == BM * BK, "A tile must split evenly");
  static_assert(B_BLK * NT * 16 == BK * BN, "B tile must split evenly");
};

__device__ __forceinline__ float4 ld4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// The kernel without epilogue stores C block by block during its last k-tile
// (kernel's ES path) when set.  Against storing after the last k-tile (same
// box, three runs each): 16 x 1024^3 batched 248.1 -> 244.4 us (+1.5%),
// 16384 x 4096 x 512 +2.4%, 4096 x 4096 x 1024 +1.6%, 8192^3 +0.4%, 4096^3
// +0.3%, 4000^3 (float4 guards) +0.7%, 2000 x 2000 x 95 and 4095 x 4096 x 33
// (scalar guards) +6% and +4%.
constexpr bool kEarlyStore = true;

template <int BM, int BN, int BK, bool CHECK, bool TB, bool EPI, bool V4 = false, bool KF = false, bool HY = false>
__global__ __launch_bounds__((EPI && BM == 256 && BN == 256) ? 512 : 256) void sgemm_mfma_kernel(
    int M, int N, int K, const float* __restrict__ A, int lda, long long sA,
    const float* __restrict__ B, int ldb, long long sB, float* __restrict__ C,
    int ldc, long long sC, int tiles_m, int tiles_n, const float* __restrict__ bias, int act,
    int hy_ndp, int hy_r, int hy_kt, float* __restrict__ hy_P, long long sAz, long long sBz, long long sCz) {
  using G = Cfg<BM, BN, BK, EPI && BM == 256 && BN == 256>;
  constexpr int LDK = G::LDK;
  extern __shared__ float4 smem4[];
  float* smem = reinterpret_cast<float*>(smem4);
  float* As = smem;                      // [2][BM][LDK]
  float* Bs = smem + 2 * BM * LDK;       // [2][BN][LDK], k-contiguous

  // ---- tile mapping (XCD-aware, grouped) ----
  const int ntiles = tiles_m * tiles_n;
  int p = blockIdx.x;
  long long bz = blockIdx.y;
  bool by_xcd = false;  // batches: (batch, tile) slots remapped XCD-contiguously
  if constexpr (!HY && !CHECK) {
    // Workgroups are dispatched round-robin over the 8 XCDs in linear id order (x fastest), so
    // a batch's tiles were spread over all eight L2s.  Each XCD takes a contiguous run of the
    // (batch, tile) slots instead: whole batches where a batch's tiles divide the run, each
    // batch's A and B then read into one L2.  Same box, three runs each (us): 16 x 1024^3
    // 248.5-251.0 -> 246.9-247.3, 8 x 1024^3 130.3-130.8 -> 127.4-127.8, 24 x 1024^3
    // 388-399 -> 381-383, 64 x 512^3 135.1-136.0 -> 132.4-133.1, 32 x 1024 x 1024 x 512 +0.9%,
    // 4 x 2048 x 2048 x 1024 +1%, 16 x 1024 x 1024 x 4096 unchanged.  Unguarded loads only: in
    // the float4-guarded 256 x 256 instantiations it doubled the k-loop's code and moved its
    // load waits.  Split-K grids (slices in z) keep the dispatch order: remapped the same way
    // they measured even or slower (1024 x 1024 x 2048 43.3-43.6 -> 44.3-44.4 us).
    const long long slots = (long long)gridDim.x * gridDim.y;
    if (gridDim.y > 1 && gridDim.z == 1 && (slots & 7) == 0) {
      const long long L = (long long)blockIdx.y * gridDim.x + blockIdx.x;
      const long long q = (L & 7) * (slots >> 3) + (L >> 3);
      bz = q / gridDim.x;
      p = (int)(q - bz * gridDim.x);
      by_xcd = true;
    }
  }
  int lt = p;
  bool tail = false;  // HY: this workgroup computes one k-slice of one of the last hy_r tiles
  int hy_slot = 0, hy_slice = 0;
  if constexpr (!HY) {
    if ((ntiles & 7) == 0 && !by_xcd) lt = (p & 7) * (ntiles >> 3) + (p >> 3);
  } else {
    // whole tiles 0 .. hy_ndp - 1 first (hy_ndp fills whole rounds), XCD-contiguous; then
    // the k-slices of tiles hy_ndp .. hy_ndp + hy_r - 1, slice-major and XCD-contiguous,
    // so that an XCD's workgroups run neighbouring tiles over the same k range
    if (p < hy_ndp) {
      if ((hy_ndp & 7) == 0) lt = (p & 7) * (hy_ndp >> 3) + (p >> 3);
    } else {
      const int nt = (int)gridDim.x - hy_ndp;
      int q = p - hy_ndp;
      if ((nt & 7) == 0) q = (q & 7) * (nt >> 3) + (q >> 3);
      hy_slice = q / hy_r;
      hy_slot = q - hy_slice * hy_r;
      lt = hy_ndp + hy_slot;
      tail = true;
    }
  }
  constexpr int GROUP = 8;
  const int group_size = GROUP * tiles_n;
  const int g = lt / group_size;
  const int first_m = g * GROUP;
  const int gm = min(tiles_m - first_m, GROUP);
  const int within = lt - g * group_size;
  const int tile_m = first_m + within % gm;
  const int tile_n = within / gm;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  A += bz * sA;
  B += bz * sB;
  C += bz * sC;
  if (gridDim.z > 1) {  // split over k: blockIdx.z is the slice (its A, B offset and partial)
    const long long zz = blockIdx.z;
    A += zz * sAz;
    B += zz * sBz;
    C += zz * sCz;
  }
  if constexpr (HY) {
    if (tail) {  // k-tiles hy_slice * hy_kt .. + hy_kt - 1, as a product of K = hy_kt * BK
      const long long k0 = (long long)hy_slice * hy_kt * BK;
      A += k0;
      B += TB ? k0 : k0 * ldb;
      K = hy_kt * BK;
    }
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 31, lh = lane >> 5;
  const int wm = (wave / G::WN) * (BM / 2);
  const int wn = (wave % G::WN) * (BN / G::WN);

  // ---- global -> register staging ----
  // A: float4 f covers row (tid / (BK/4)) + f * (NT / (BK/4)), cols
  //    4*(tid % (BK/4)) .. +3 of the k-tile.
  constexpr int A_TPR = BK / 4;                 // threads per A row
  constexpr int A_RSTEP = G::NT / A_TPR;     // rows per float4 round
  const int a_r = tid / A_TPR, a_c = (tid % A_TPR) * 4;
  // B: 4x4 block q covers k rows 4*kq .. +3 and n cols 4*nq .. +3 where
  //    blk = tid + q*NT, kq = blk % (BK/4), nq = blk / (BK/4).  The 8
  //    lanes of an LDS store phase then write one row's 8 consecutive float4
  //    (128 contiguous bytes, no bank conflict); with nq varying fastest
  //    they wrote rows 4 apart, 16-way conflicted (measured: 130.5 vs 134.3
  //    TFLOP/s at 4096^3).  A global load still covers whole 128-byte lines.
  constexpr int B_KQ = BK / 4;
  // BROW (unguarded [K][N] B, 256-row tiles): B is kept row-major in LDS ([k][LDN], rows
  // copied with 128-bit loads and stores like A) and its fragments are read as four 32-bit
  // values per block.  The 4 x 4 transpose through registers it replaces left the staged
  // registers permuted across the loop's back edge, so every iteration ended copying them
  // behind a wait for all of the next tile's loads.  Same box, two runs each, TFLOP/s: 4096^3
  // 145.4 -> 147.1, 16 x 1024^3 batched 135.7 -> 138.5, 8192 x 8192 x 2048 144.2 -> 145.8,
  // 4096 x 4096 x 1024 138.2 -> 139.3, 3072^3 (256 x 128 tiles) 137.0 -> 137.8; the 128 x 128
  // tile, with 16 MFMAs a chunk for its 8 extra LDS reads, lost (2048 x 2048 x 4096 136.1 ->
  // 121.5) and keeps the transpose.  (The compiler pairs those reads into ds_read2_b32; with the
  // scheduling groups counting the pairs its loop waits only for the previous tile's loads, and
  // it measured even: 128 x 11008 x 4096 109.2-110.3 -> 108.2 us, 2048 x 2048 x 4096 250.2 ->
  // 252.8, 2048 x 2048 x 1024 68.9 -> 68.3, 1024 x 1024 x 4096 unchanged.)
  // The 64 x 64 small tile (BK 64) takes the row layout too, with its fragments' B values counted
  // as read pairs in the scheduling groups (the compiler merges them into ds_read2_b32; counted
  // singly they overfill its 4-MFMA chunks): its loop had ended copying the staged B registers
  // behind a wait for the next tile's loads.  Same box, two runs each (us): 256^3 8.6-8.7 ->
  // 8.0-8.1, 512^3 13.5-13.7 -> 13.4, 768^3 19.1-19.2 -> 18.8-18.9, 1024^3 24.4 -> 24.5-24.6,
  // 1024 x 2048 x 1024 even.
  constexpr bool BROW = !TB && !CHECK && (BM == 256 || (BM == 64 && BN == 64));
  constexpr int LDN = BN + 4;                   // padded [k] row of B (floats)
  constexpr int B_TPR = BN / 4;                 // threads per B row
  constexpr int B_RSTEP = G::NT / B_TPR;     // B rows per float4 round
  static_assert(!BROW || (BK * LDN <= BN * LDK && 4 * G::B_BLK * B_RSTEP == BK), "B row layout");
  const int b_r = tid / B_TPR, b_c = (tid % B_TPR) * 4;

  float4 ra[G::A_F4];
  float4 rb[G::B_BLK][4];  // TB: rb[q][e] is float4 number 4q + e of the [n][k] tile rows

  // V4 (with CHECK): K, N, the leading dimensions and strides are multiples
  // of 4, A and B 16-byte aligned, and each operand's extent below 2 GiB.  A
  // float4 then lies wholly inside or wholly outside the matrix, and the
  // guarded load is one range-checked buffer load: outside, its offset is
  // set past the resource's end and the hardware returns zeros.  The guard
  // acts on the address only, so nothing waits on the data before the LDS
  // store a tile later (a select on the loaded value made every load's
  // latency exposed: 4000^3 at 87 TFLOP/s against 97 for scalar guards).
  // Offsets stay below 2^32: kBad plus at most 2^31 - 1 (the host checks that
  // (K + BK) rows of a [K][N] B fit in 2^31 bytes).  A row (column) outside
  // the matrix keeps kBad in its base offset, so adding the column of the
  // load leaves it past the end.  Only the k check remains: a [K][N] B never
  // needs it (rows from K on are past the resource's end), and with K a
  // multiple of BK (KF) no load of A or of a [N][K] B reaches past K either,
  // so those loads are one add.  Against the compare-and-select on every
  // load (same box, clocks settled): 4100 x 4100 x 4096 and 6000 x 6000 x
  // 3200 (128 x 128 tile) +3.2%, 3000 x 3000 x 1000 (ragged K, only the
  // [K][N] check gone) +2.3%, 4000^3 +1.7%, 2000 x 8000 x 4096 +1.2%.
  constexpr unsigned kBad = 0x80000000u;  // an offset past every resource's end
  // (unused, and removed, unless CHECK && V4)
  const int a_bytes = (int)(((long long)(M - 1) * lda + K) * 4);
  const int b_bytes = TB ? (int)(((long long)(N - 1) * ldb + K) * 4) : (int)(((long long)(K - 1) * ldb + N) * 4);
  const __amdgpu_buffer_rsrc_t ra_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0, a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0, b_bytes, 0x00020000);
  unsigned aoff[G::A_F4], boff[TB ? 4 * G::B_BLK : G::B_BLK];
  if constexpr (CHECK && V4) {
#pragma unroll
    for (int f = 0; f < G::A_F4; ++f) {
      const int gr = m0 + a_r + f * A_RSTEP;
      aoff[f] = gr < M ? (unsigned)gr * (unsigned)lda * 4u : kBad;  // row start, or kBad
    }
    if constexpr (TB) {
#pragma unroll
      for (int f = 0; f < 4 * G::B_BLK; ++f) {
        const int gr = n0 + a_r + f * A_RSTEP;
        boff[f] = gr < N ? (unsigned)gr * (unsigned)ldb * 4u : kBad;
      }
    } else {
#pragma unroll
      for (int q = 0; q < G::B_BLK; ++q) {
        const int gn = n0 + 4 * ((tid + q * G::NT) / B_KQ);
        boff[q] = gn < N ? (unsigned)gn * 4u : kBad;  // column, or kBad
      }
    }
  }
  auto ld4_rs = [&](__amdgpu_buffer_rsrc_t rs, unsigned off) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
  };
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int f = 0; f < G::A_F4; ++f) {
      const int r = a_r + f * A_RSTEP;
      const int gr = m0 + r, gc = k0 + a_c;
      if (!CHECK) {
        ra[f] = ld4(A + (long long)gr * lda + gc);
      } else if (V4) {
        ra[f] = ld4_rs(ra_rs, KF ? aoff[f] + (unsigned)gc * 4u
                                : (aoff[f] != kBad && gc < K) ? aoff[f] + (unsigned)gc * 4u : kBad);
      } else {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          t[e] = (gr < M && gc + e < K) ? A[(long long)gr * lda + gc + e] : 0.0f;
        ra[f] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
    if constexpr (TB) {
      // rows of B^T are rows of the [n][k] input: same pattern as A
#pragma unroll
      for (int f = 0; f < 4 * G::B_BLK; ++f) {
        const int r = a_r + f * A_RSTEP;
        const int gr = n0 + r, gc = k0 + a_c;
        if (!CHECK) {
          rb[f >> 2][f & 3] = ld4(B + (long long)gr * ldb + gc);
        } else if (V4) {
          rb[f >> 2][f & 3] = ld4_rs(rb_rs, KF ? boff[f] + (unsigned)gc * 4u
                                           : (boff[f] != kBad && gc < K) ? boff[f] + (unsigned)gc * 4u : kBad);
        } else {
          float t[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            t[e] = (gr < N && gc + e < K) ? B[(long long)gr * ldb + gc + e] : 0.0f;
          rb[f >> 2][f & 3] = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
    } else if constexpr (BROW) {
#pragma unroll
      for (int f = 0; f < 4 * G::B_BLK; ++f)
        rb[f >> 2][f & 3] = ld4(B + (long long)(k0 + b_r + f * B_RSTEP) * ldb + n0 + b_c);
    } else {
#pragma unroll
      for (int q = 0; q < G::B_BLK; ++q) {
        const int blk = tid + q * G::NT;
        const int kq = blk % B_KQ, nq = blk / B_KQ;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gk = k0 + 4 * kq + e, gn = n0 + 4 * nq;
          if (!CHECK) {
            rb[q][e] = ld4(B + (long long)gk * ldb + gn);
          } else if (V4) {
            rb[q][e] = ld4_rs(rb_rs, (unsigned)gk * (unsigned)ldb * 4u + boff[q]);
          } else {
            float t[4];
#pragma unroll
            for (int c = 0; c < 4; ++c)
              t[c] = (gk < K && gn + c < N) ? B[(long long)gk * ldb + gn + c] : 0.0f;
            rb[q][e] = make_float4(t[0], t[1], t[2], t[3]);
          }
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    float* as = As + buf * BM * LDK;
    float* bs = Bs + buf * BN * LDK;
#pragma unroll
    for (int f = 0; f < G::A_F4; ++f) {
      const int r = a_r + f * A_RSTEP;
      *reinterpret_cast<float4*>(as + r * LDK + a_c) = ra[f];
    }
    if constexpr (TB) {
#pragma unroll
      for (int f = 0; f < 4 * G::B_BLK; ++f) {
        const int r = a_r + f * A_RSTEP;
        *reinterpret_cast<float4*>(bs + r * LDK + a_c) = rb[f >> 2][f & 3];
      }
      return;
    }
    if constexpr (BROW) {
#pragma unroll
      for (int f = 0; f < 4 * G::B_BLK; ++f)
        *reinterpret_cast<float4*>(bs + (b_r + f * B_RSTEP) * LDN + b_c) = rb[f >> 2][f & 3];
      return;
    }
#pragma unroll
    for (int q = 0; q < G::B_BLK; ++q) {
      const int blk = tid + q * G::NT;
      const int kq = blk % B_KQ, nq = blk / B_KQ;
      // transpose the 4(k) x 4(n) block: column c of rb -> LDS row n
      float* base = bs + (4 * nq) * LDK + 4 * kq;
      *reinterpret_cast<float4*>(base + 0 * LDK) =
          make_float4(rb[q][0].x, rb[q][1].x, rb[q][2].x, rb[q][3].x);
      *reinterpret_cast<float4*>(base + 1 * LDK) =
          make_float4(rb[q][0].y, rb[q][1].y, rb[q][2].y, rb[q][3].y);
      *reinterpret_cast<float4*>(base + 2 * LDK) =
          make_float4(rb[q][0].z, rb[q][1].z, rb[q][2].z, rb[q][3].z);
      *reinterpret_cast<float4*>(base + 3 * LDK) =
          make_float4(rb[q][0].w, rb[q][1].w, rb[q][2].w, rb[q][3].w);
    }
  };

  f32x16 acc[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Fragments are double-buffered by chunk (8 k): the LDS reads of chunk c + 1
  // are issued before the MFMAs of chunk c, the next tile's LDS stores go out
  // with chunk NC - 2, and the one barrier per tile sits before the MFMAs of
  // the last chunk, whose fragments are already in registers.  The reads of
  // the next tile's chunk 0 then overlap those MFMAs.  Buffer cur ^ 1 was
  // last read before the previous tile's barrier, so storing it after that
  // barrier is safe; its reads come after this tile's barrier.
  constexpr int NC = BK / 8;
  static_assert(NC % 2 == 0 && NC >= 2, "chunk count must be even");
  float4 fa[2][G::TM], fb[2][G::TN];
  auto read_frags = [&](int buf, int c, float4 (&a)[G::TM], float4 (&b)[G::TN]) {
    const float* as = As + buf * BM * LDK + (wm + li) * LDK + 4 * lh + 8 * c;
#pragma unroll
    for (int i = 0; i < G::TM; ++i) a[i] = *reinterpret_cast<const float4*>(as + i * 32 * LDK);
    if constexpr (BROW) {
      // B[k = 8c + 4lh + s][n = wn + 32j + li], s = 0..3: four rows of the [k][n] tile
      const float* bs = Bs + buf * BN * LDK + (8 * c + 4 * lh) * LDN + wn + li;
#pragma unroll
      for (int j = 0; j < G::TN; ++j)
        b[j] = make_float4(bs[j * 32], bs[LDN + j * 32], bs[2 * LDN + j * 32], bs[3 * LDN + j * 32]);
    } else {
      const float* bs = Bs + buf * BN * LDK + (wn + li) * LDK + 4 * lh + 8 * c;
#pragma unroll
      for (int j = 0; j < G::TN; ++j) b[j] = *reinterpret_cast<const float4*>(bs + j * 32 * LDK);
    }
  };
  auto mfma_chunk = [&](const float4 (&a)[G::TM], const float4 (&b)[G::TN]) {
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
      for (int j = 0; j < G::TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
  };

  const int nk = (K + BK - 1) / BK;
  if (nk > 0) {
    load_tile(0);
    store_tile(0);
    load_tile(min(1, nk - 1) * BK);
  }
  __syncthreads();
  if (nk > 0) read_frags(0, 0, fa[0], fb[0]);

  // Branch-free body (one basic block the scheduler can interleave): the
  // last iteration reloads the last tile into the buffer no one reads again.
  // The order is pinned with scheduling groups (mask 0x008 MFMA, 0x100 LDS
  // read, 0x200 LDS write): left alone, the scheduler sank the global loads
  // to the end of the body behind a vmcnt(0) and clustered the LDS traffic.
  constexpr int NR = G::TM + (BROW ? (BM == 64 ? 2 : 4) : 1) * G::TN;       // LDS reads per chunk
  constexpr int NW = G::A_F4 + 4 * G::B_BLK;               // LDS stores per tile
  constexpr int NM = 4 * G::TM * G::TN;                    // MFMAs per chunk
  // the small tile (one MFMA block per wavefront) has too few MFMAs in a chunk to pin its
  // stores between them; they go where the scheduler puts them within their chunk
  constexpr bool PIN = NM >= NR + NW;
  constexpr int MPW = !PIN ? 0 : (NM - NR) / NW >= 2 ? 2 : 1;  // MFMAs after each store
  static_assert(NM >= NR + MPW * NW, "chunk too small to cover its LDS traffic");
  // ES: the last k-tile is peeled (below) so that C leaves block by block
  // (the 256 x 128 tile in every load mode, and the scalar-guarded 128 x 128 tile: the
  // float4-guarded and unguarded 128 x 128 tiles measured 0.2-1.1% slower with it).  The
  // 256 x 256 tile stores after the loop: with B row-major in LDS, holding the last tile's four
  // chunks of fragments spilled 64-101 VGPRs to scratch in every load mode, and without the peel
  // it spills none.  Same box, two runs each (us, peeled -> not): 16 x 1024^3 246.3-247.9 ->
  // 243.7-243.8, 32 x 1024 x 1024 x 512 264.5 -> 254.5-254.8, 16384 x 4096 x 512 518-520 ->
  // 502, 4096 x 4096 x 1024 247.3-247.5 -> 243.9-244.5, 4095 x 4096 x 33 (scalar guards)
  // 38.9-39.0 -> 35.0, 4096^3 and 8192^3 even, 4000^3 (float4 guards) 922.5-924.7 ->
  // 925.6-927.9.
  constexpr bool ES = kEarlyStore && !EPI && !HY && G::TN % 2 == 0 && !(BM == 256 && BN == 256) &&
                      (BM == 256 || (CHECK && !V4));
  const int nloop = ES ? nk - 1 : nk;
  for (int t = 0; t < nloop; ++t) {
    const int cur = t & 1;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c == NC - 1) __syncthreads();
      read_frags(c == NC - 1 ? cur ^ 1 : cur, (c + 1) % NC, fa[(c + 1) & 1], fb[(c + 1) & 1]);
      if (c == NC - 2) {
        store_tile(cur ^ 1);
        load_tile(min(t + 2, nk - 1) * BK);
      }
      mfma_chunk(fa[c & 1], fb[c & 1]);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      if (PIN && c == NC - 2) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, MPW, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NM - NR - MPW * NW, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if constexpr (ES) {
    // The last k-tile block-major: its four chunks' fragments at once (chunk 0 is
    // already in fa[0] / fb[0]; nothing writes LDS any more), then two 32 x 32
    // blocks' 32 MFMAs at a time, each pair stored while the next pair's MFMAs
    // run, so C goes out during the last k-tile instead of after it.
    if (nk > 0) {
      const int cur = (nk - 1) & 1;
      float4 la[NC][G::TM], lb[NC][G::TN];
#pragma unroll
      for (int i = 0; i < G::TM; ++i) la[0][i] = fa[0][i];
#pragma unroll
      for (int j = 0; j < G::TN; ++j) lb[0][j] = fb[0][j];
#pragma unroll
      for (int c = 1; c < NC; ++c) read_frags(cur, c, la[c], lb[c]);
      constexpr int NP = G::TM * G::TN / 2;  // block pairs (i, 2q), (i, 2q + 1)
      auto mm_pair = [&](int pr) {
        const int i = pr / (G::TN / 2), j = 2 * (pr % (G::TN / 2));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].x, lb[c][j].x, acc[i][j], 0, 0, 0);
          acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].x, lb[c][j + 1].x, acc[i][j + 1], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].y, lb[c][j].y, acc[i][j], 0, 0, 0);
          acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].y, lb[c][j + 1].y, acc[i][j + 1], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].z, lb[c][j].z, acc[i][j], 0, 0, 0);
          acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].z, lb[c][j + 1].z, acc[i][j + 1], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].w, lb[c][j].w, acc[i][j], 0, 0, 0);
          acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(la[c][i].w, lb[c][j + 1].w, acc[i][j + 1], 0, 0, 0);
        }
      };
      auto st_pair = [&](int pr) {
        const int i = pr / (G::TN / 2), j = 2 * (pr % (G::TN / 2));
#pragma unroll
        for (int jj = j; jj < j + 2; ++jj) {
          const int col = n0 + wn + jj * 32 + li;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (!CHECK || (row < M && col < N)) C[(long long)row * ldc + col] = acc[i][jj][r];
          }
        }
      };
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int pr = 0; pr < NP; ++pr) {
        mm_pair(pr);
        if (pr > 0) st_pair(pr - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      st_pair(NP - 1);
      return;
    }
    // K = 0: no k-tile to peel; the epilogue below stores the zero accumulators
  }

  // ---- epilogue: value r of lane l is row 8*(r/4) + 4*lh + r%4, col li ----
  if constexpr (HY) {
    if (tail) {  // the slice's sums, a whole BM x BN tile, into its slot of the partials
      float* Pt = hy_P + ((long long)hy_slice * hy_r + hy_slot) * (BM * BN);
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            Pt[(wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)) * BN + wn + j * 32 + li] = acc[i][j][r];
      return;
    }
  }
  if constexpr (!EPI) {
#pragma unroll
    for (int i = 0; i < G::TM; ++i) {
#pragma unroll
      for (int j = 0; j < G::TN; ++j) {
        const int col = n0 + wn + j * 32 + li;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (!CHECK || (row < M && col < N)) C[(long long)row * ldc + col] = acc[i][j][r];
        }
      }
    }
  } else {
    // bias and the activation are uniform over the launch (no divergence); one 32 x 32
    // block at a time, so only 16 accumulators are out of the AGPRs at once
#pragma unroll
    for (int j = 0; j < G::TN; ++j) {
      const int col = n0 + wn + j * 32 + li;
      const float bj = bias ? (!CHECK || col < N ? bias[col] : 0.0f) : 0.0f;
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          float v = acc[i][j][r] + bj;
          v = bch::activate(v, act);
          if (!CHECK || (row < M && col < N)) C[(long long)row * ldc + col] = v;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

template <int BM, int BN, int BK, bool CHECK, bool TB, bool EPI, bool V4 = false, bool KF = false>
hipError_t launch_tiles(hipStream_t s, int batch, int m, int n, int k,
                        const float* A, int lda, long long sA, const float* B,
                        int ldb, long long sB, float* C, int ldc, long long sC,
                        const float* bias, int act, int nz = 1, long long sAz = 0, long long sBz = 0,
                        long long sCz = 0) {
  using G = Cfg<BM, BN, BK, EPI && BM == 256 && BN == 256>;
  const int tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  const size_t lds = sizeof(float) * G::LDS_FLOATS;
  auto kern = sgemm_mfma_kernel<BM, BN, BK, CHECK, TB, EPI, V4, KF>;
  hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(kern), (int)lds);
  if (e != hipSuccess) return e;
  if (batch > 65535 || nz > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3(tm * tn, batch, nz), dim3(G::NT), lds, s, m, n, k,
                     A, lda, sA, B, ldb, sB, C, ldc, sC, tm, tn, bias, act, 0, 0, 0, nullptr, sAz, sBz, sCz);
  return hipGetLastError();
}

// The hybrid launch (batch 1, K a multiple of BK): ndp whole tiles, then r tiles in
// S k-slices of kt k-tiles each into P (see HybPlan).
template <int BM, int BN, int BK, bool CHECK, bool TB, bool EPI, bool V4, bool KF>
hipError_t launch_hyb_tiles(hipStream_t s, int m, int n, int k, const float* A, int lda, const float* B, int ldb,
                            float* C, int ldc, const float* bias, int act, int ndp, int r, int S, int kt, float* P) {
  using G = Cfg<BM, BN, BK, EPI && BM == 256 && BN == 256>;
  const int tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  const size_t lds = sizeof(float) * G::LDS_FLOATS;
  auto kern = sgemm_mfma_kernel<BM, BN, BK, CHECK, TB, EPI, V4, KF, true>;
  hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(kern), (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(ndp + r * S), dim3(G::NT), lds, s, m, n, k, A, lda, 0LL, B, ldb, 0LL, C, ldc,
                     0LL, tm, tn, bias, act, ndp, r, kt, P, 0LL, 0LL, 0LL);
  return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

constexpr int kBK = 32;

// Tile choice: the tile with the least modelled time, rounds x tile area /
// efficiency, where a round is one workgroup per CU (one 256x256 workgroup
// fits a CU; the smaller tiles are timed at full rounds) and the efficiencies
// are the tiles' measured rates at whole rounds relative to 256x256 (TFLOP/s
// on MI355X: 256x256 145 at 4096^3, 256x128 140 at 8192 x 1024 x 8192,
// 128x128 128 at 2048^3).  The largest tile that still fills every CU is
// what this gives when the counts come out even; otherwise a part-filled last
// round of large tiles can cost more than more rounds of smaller ones
// (6144^3: three rounds of 256x256, 107 TFLOP/s).
enum class Tile { k256x256, k256x128, k128x128 };

struct TileOpt { Tile t; int bm, bn; double eff; };
constexpr TileOpt kTileOpts[] = {{Tile::k256x256, 256, 256, 1.0}, {Tile::k256x128, 256, 128, 0.966},
                                 {Tile::k128x128, 128, 128, 0.92}};

Tile pick_tile(int batch, int m, int n) {
  const long long cu = bch::device_cu_count();
  Tile best = Tile::k256x256;
  double best_cost = 0.0;
  for (const TileOpt& o : kTileOpts) {
    const long long tiles = (long long)batch * ((m + o.bm - 1) / o.bm) * ((n + o.bn - 1) / o.bn);
    const double cost = (double)((tiles + cu - 1) / cu) * o.bm * o.bn / o.eff;
    if (o.t == Tile::k256x256 || cost < best_cost * 0.999) {
      best = o.t;
      best_cost = cost;
    }
  }
  return best;
}

int tile_m(Tile t) { return t == Tile::k128x128 ? 128 : 256; }
int tile_n(Tile t) { return t == Tile::k256x256 ? 256 : 128; }

bool fast_ok(Tile t, int m, int n, int k, const float* A, int lda, long long sA, const float* B, int ldb,
             long long sB) {
  return m % tile_m(t) == 0 && n % tile_n(t) == 0 && k % kBK == 0 && lda % 4 == 0 && ldb % 4 == 0 &&
         sA % 4 == 0 && sB % 4 == 0 && aligned16(A) && aligned16(B);
}

// Guarded loads as whole float4: K and N multiples of 4 (a float4 along k, or
// along n for a [k][n] B, is then wholly inside or wholly outside), leading
// dimensions and batch strides multiples of 4, A and B 16-byte aligned, and
// each operand's extent (per batch) below 2 GiB for the 32-bit buffer offsets.
bool vec4_ok(bool transb, int m, int n, int k, const float* A, int lda, long long sA, const float* B, int ldb,
             long long sB) {
  const long long a_bytes = ((long long)(m - 1) * lda + k) * 4;
  // a [K][N] B's loads reach up to row K + kBK - 1 (past the resource's end, read as zeros)
  const long long b_bytes = (transb ? (long long)(n - 1) * ldb + k : (long long)(k + kBK) * ldb) * 4;
  return k >= 4 && k % 4 == 0 && n % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && sA % 4 == 0 && sB % 4 == 0 &&
         aligned16(A) && aligned16(B) && a_bytes < (1LL << 31) && b_bytes < (1LL << 31);
}

// k slices in grid.z (the split-K launch): slice z adds z * (sA, sB, sC) to the batch's operands
struct ZSplit {
  int nz = 1;
  long long sA = 0, sB = 0, sC = 0;
};

template <bool CHECK, bool TB, bool EPI, bool V4, bool KF = false>
hipError_t launch_tile(Tile t, hipStream_t s, int batch, int m, int n, int k, const float* A, int lda,
                       long long sA, const float* B, int ldb, long long sB, float* C, int ldc, long long sC,
                       const float* bias, int act, const ZSplit& z) {
  switch (t) {
    case Tile::k256x256:
      return launch_tiles<256, 256, kBK, CHECK, TB, EPI, V4, KF>(s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                                             bias, act, z.nz, z.sA, z.sB, z.sC);
    case Tile::k256x128:
      return launch_tiles<256, 128, kBK, CHECK, TB, EPI, V4, KF>(s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                                             bias, act, z.nz, z.sA, z.sB, z.sC);
    default:
      return launch_tiles<128, 128, kBK, CHECK, TB, EPI, V4, KF>(s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                                             bias, act, z.nz, z.sA, z.sB, z.sC);
  }
}

// mode 0: unguarded; 1: guarded float4 loads; 2: guarded scalar loads
template <bool TB, bool EPI>
hipError_t launch_tile_any(int mode, Tile t, hipStream_t s, int batch, int m, int n, int k, const float* A,
                           int lda, long long sA, const float* B, int ldb, long long sB, float* C, int ldc,
                           long long sC, const float* bias, int act, const ZSplit& z = ZSplit{}) {
  if (mode == 0)
    return launch_tile<false, TB, EPI, false>(t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act, z);
  if (mode == 1 && k % kBK == 0)
    return launch_tile<true, TB, EPI, true, true>(t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act,
                                                  z);
  if (mode == 1)
    return launch_tile<true, TB, EPI, true>(t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act, z);
  return launch_tile<true, TB, EPI, false>(t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act, z);
}

const char* tile_name(Tile t, int mode) {
  static const char* const names[3][3] = {
      {"sgemm_mfma_kernel<256,256,32,false>", "sgemm_mfma_kernel<256,256,32,true,v4>", "sgemm_mfma_kernel<256,256,32,true>"},
      {"sgemm_mfma_kernel<256,128,32,false>", "sgemm_mfma_kernel<256,128,32,true,v4>", "sgemm_mfma_kernel<256,128,32,true>"},
      {"sgemm_mfma_kernel<128,128,32,false>", "sgemm_mfma_kernel<128,128,32,true,v4>", "sgemm_mfma_kernel<128,128,32,true>"}};
  return names[static_cast<int>(t)][mode];
}

// ---- split-K for shapes whose tiles fill less than one round ----
// K is cut into S slices of whole k-tiles; the slices run as one launch of
// the tile kernel with the slice in grid.z (batch b, slice j: A + b sA + j kc,
// B + b sB + j kc rows -- or columns for B given as [n][k] -- into P[b][j],
// an m x n partial), then sgemm_splitk_reduce sums the S partials of each
// output in slice order (deterministic) and applies the epilogue.  Batches
// split the same way when all of their tiles together fill less than a
// round (4 x 512 x 512 x 4096: 64 tiles).  S is the modelled fastest:
// rounds(tiles x S) x k-tiles per slice x the tile's k-tile time (7.4 us for
// 256 x 256 at full rate, scaled by area / efficiency), plus the partials'
// round trip ((2S + 1) M N floats at 5 TB/s) and a launch; S divides the
// k-tile count, leaves at least kSplitMinKt k-tiles per slice, and its
// partials fit the cap.  The plan is made against a fixed cap, not the
// workspace at hand, so a shape always rounds the same way through
// bch_sgemm; bch_sgemm_noalloc plans against its 16 MiB scratch and can take
// fewer slices (within tolerance of bch_sgemm).  Several rounds of slices
// can beat one part-filled round: 128 x 11008 x 4096 on 86 tiles of 128 x
// 128 takes 8 slices in 3 rounds rather than 2 in one.  Measured at 1024^3
// (64 tiles of 128 x 128): 64.8 us on 64 CUs without the split.
constexpr size_t kSplitWsMax = (size_t)256 << 20;
constexpr size_t kSplitWsSmall = (size_t)16 << 20;  // bch_sgemm_noalloc's fixed scratch
constexpr int kSplitMinKt = 8;  // k-tiles per slice at least

int split_slices(int batch, int m, int n, int k, size_t cap = kSplitWsMax, double* cost_us = nullptr) {
  if (batch < 1 || k <= 0 || k % kBK != 0) return 1;
  const long long cu = bch::device_cu_count();
  const Tile t = pick_tile(batch, m, n);
  const long long tiles =
      (long long)batch * ((m + tile_m(t) - 1) / tile_m(t)) * ((n + tile_n(t) - 1) / tile_n(t));
  if (tiles >= cu) return 1;  // whole rounds: the data-parallel tiling or the hybrid plan
  double eff = 1.0;
  for (const TileOpt& o : kTileOpts)
    if (o.t == t) eff = o.eff;
  const double tk = 7.4 * tile_m(t) * tile_n(t) / 65536.0 / eff;  // us per k-tile of this tile
  const double mn = (double)batch * m * n * sizeof(float);
  const int nk = k / kBK;
  double best = nk * tk;
  int bs = 1;
  for (int sl = 2; nk / sl >= kSplitMinKt; ++sl) {
    if (nk % sl != 0) continue;
    if ((size_t)sl * batch * m * n * sizeof(float) > cap) break;
    const double cost = (double)((tiles * sl + cu - 1) / cu) * (nk / sl) * tk + (2.0 * sl + 1.0) * mn / 5e6 + 2.0;
    if (cost < best) {
      best = cost;
      bs = sl;
    }
  }
  if (cost_us) *cost_us = best;
  return bs;
}

// ---- small shapes: 64 x 64 x 64 tiles ----
// Where the planned tiles fill less than one round, 64 x 64 tiles (each wavefront one 32 x 32
// MFMA block; k-tiles of 64 so that a tile's loads split evenly over the 256 threads) put 16x
// the workgroups of the 128 x 128 tiling on the CUs, with no k split, partials or reduce
// launch.  A 64 x 64 x 64 k-tile takes ~1.32 us at any count of tiles up to a round (256^3 to
// 1024^3; 63% of the matrix cores' rate, against 92% for 128 x 128); two workgroups share a CU
// (70 KB of LDS each) at ~2.29 us per k-tile of both.  Taken when its modelled time, rounds x
// k-tiles x that time, is under 0.9 of the split-K plan's; unguarded loads only (m, n, k
// multiples of 64, aligned operands), else the usual path.  Same box, two runs each, against
// the split-K plan: 256^3 19.4 -> 8.8 us, 512^3 23.0 -> 13.9, 768^3 25.8 -> 19.3, 1024^3 28.3
// -> 24.4, 1024 x 2048 x 1024 43.9 -> 40.1 (two per CU); where split-K stays ahead the model
// keeps it (1024 x 1024 x 4096 74 against 89 us, 1024 x 1024 x 2048 43.5 against 47.6, 512 x
// 1024 x 2048 28.7 against 46.9).
constexpr int kSmallBK = 64;
constexpr double kSmallKtUs = 1.32;   // one workgroup per CU
constexpr double kSmallKt2Us = 2.29;  // two per CU, both k-tiles

bool small_tile_plan(int batch, int m, int n, int k) {
  if (batch < 1 || m % 64 != 0 || n % 64 != 0 || k <= 0 || k % kSmallBK != 0) return false;
  const long long cu = bch::device_cu_count();
  const Tile t = pick_tile(batch, m, n);
  const long long tiles =
      (long long)batch * ((m + tile_m(t) - 1) / tile_m(t)) * ((n + tile_n(t) - 1) / tile_n(t));
  if (tiles >= cu) return false;
  double cur = 0.0;
  split_slices(batch, m, n, k, kSplitWsMax, &cur);
  const long long t64 = (long long)batch * (m / 64) * (n / 64);
  const double nk = k / kSmallBK;
  const double small = t64 <= cu ? nk * kSmallKtUs : (double)((t64 + 2 * cu - 1) / (2 * cu)) * nk * kSmallKt2Us;
  return small < 0.9 * cur;
}

bool small_tile_ok(int batch, int m, int n, int k, const float* A, int lda, long long sA, const float* B, int ldb,
                   long long sB) {
  return small_tile_plan(batch, m, n, k) && lda % 4 == 0 && ldb % 4 == 0 && sA % 4 == 0 && sB % 4 == 0 &&
         aligned16(A) && aligned16(B);
}

// C[b][m][n] = act(sum over j < S of P[b][j][m][n] (+ bias[n])) for each of `batch` matrices
// (C[b] at C + b sC); V: four columns per thread (n % 4 == 0, ldc % 4 == 0, C 16-byte aligned)
template <bool V>
__global__ __launch_bounds__(256) void sgemm_splitk_reduce(int M, int N, int S, int batch, const float* __restrict__ P,
                                                           float* __restrict__ C, int ldc, long long sC,
                                                           const float* __restrict__ bias, int act) {
  const long long per = (long long)M * N;
  const int w = V ? 4 : 1;
  const long long total = per * batch / w;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long ea = i * w;
    const long long b = ea / per, e = ea - b * per;
    const int m = (int)(e / N), n = (int)(e - (long long)m * N);
    const float* pb = P + b * S * per + e;
    float* cb = C + b * sC + (long long)m * ldc + n;
    if constexpr (V) {
      float4 acc = *reinterpret_cast<const float4*>(pb);
      for (int j = 1; j < S; ++j) {
        const float4 x = *reinterpret_cast<const float4*>(pb + j * per);
        acc.x += x.x;
        acc.y += x.y;
        acc.z += x.z;
        acc.w += x.w;
      }
      if (bias) {
        acc.x += bias[n];
        acc.y += bias[n + 1];
        acc.z += bias[n + 2];
        acc.w += bias[n + 3];
      }
      acc = make_float4(bch::activate(acc.x, act), bch::activate(acc.y, act), bch::activate(acc.z, act),
                        bch::activate(acc.w, act));
      *reinterpret_cast<float4*>(cb) = acc;
    } else {
      float acc = pb[0];
      for (int j = 1; j < S; ++j) acc += pb[j * per];
      if (bias) acc += bias[n];
      *cb = bch::activate(acc, act);
    }
  }
}

// ---- whole rounds data-parallel, the last round's tiles split over k (the hybrid plan) ----
// With T tiles on CU compute units, R = T / CU whole rounds and r = T mod CU
// tiles left over, the last round would run r workgroups of full length on
// r CUs.  Instead one launch runs the R * CU whole tiles and then the r tiles
// in S slices of equal k length (S * r <= CU), each slice's sums stored as a
// compact BM x BN tile; sgemm_tail_reduce adds each tile's S slices in slice
// order (deterministic) and applies the epilogue that the whole tiles apply
// in the kernel.  Every slice covers the same k-tiles of neighbouring tiles,
// so the slices of a round share A and B panels in L2 the way whole tiles do.
// The plan is modelled like the tile choice (k-tiles x tile area /
// efficiency per round; the partials' HBM traffic at 5 TB/s, one 256 x 256
// k-tile taking 7.4 us) and used when it beats the best data-parallel tiling
// by 3%.  It needs K a multiple of 32 and unguarded or float4-guarded loads;
// without the workspace (up to kHybWsMax) the data-parallel tiling runs.
constexpr size_t kHybWsMax = (size_t)256 << 20;

struct HybPlan {
  Tile t = Tile::k256x256;
  int S = 0, ndp = 0, r = 0, kt = 0;  // slices, whole tiles, split tiles, k-tiles per slice
};

size_t hyb_bytes(const HybPlan& h) { return (size_t)h.S * h.r * tile_m(h.t) * tile_n(h.t) * sizeof(float); }

// cost_us (nullable): the modelled time of what the tile path then runs, the hybrid plan or the
// best data-parallel tiling (7.4 us per 256 x 256 k-tile)
bool hyb_plan(int batch, int m, int n, int k, HybPlan& out, double* cost_us = nullptr) {
  if (batch != 1 || k <= 0 || k % kBK != 0 || split_slices(batch, m, n, k) > 1) return false;
  const long long cu = bch::device_cu_count();
  const int nk = k / kBK;
  double best_dp = 0.0, best = 0.0;
  bool found = false;
  for (const TileOpt& o : kTileOpts) {
    const long long T = (long long)((m + o.bm - 1) / o.bm) * ((n + o.bn - 1) / o.bn);
    const double per = o.bm * o.bn / 65536.0 / o.eff;  // one k-tile of this tile, in 256 x 256 k-tiles
    const double dp = (double)((T + cu - 1) / cu) * nk * per;
    if (best_dp == 0.0 || dp < best_dp) best_dp = dp;
    const long long R = T / cu, r = T % cu;
    if (R < 1 || r == 0) continue;
    int S = 0;
    for (int sl = 8; sl >= 2; --sl)
      if (sl * r <= cu && nk % sl == 0 && nk / sl >= kSplitMinKt &&
          (size_t)sl * r * o.bm * o.bn * sizeof(float) <= kHybWsMax) {
        S = sl;
        break;
      }
    if (S == 0) continue;
    const double cost = (double)(R * nk + nk / S) * per + (2.0 * S + 1.0) * r * (o.bm * o.bn / 65536.0) * 0.00709 + 0.3;
    if (!found || cost < best) {
      found = true;
      best = cost;
      out.t = o.t;
      out.S = S;
      out.ndp = (int)(R * cu);
      out.r = (int)r;
      out.kt = nk / S;
    }
  }
  const bool use = found && best < 0.97 * best_dp;
  if (cost_us) *cost_us = 7.4 * (use ? best : best_dp);
  return use;
}

// Modelled time (us) of a batch-1 call on the tile path: split-K, the hybrid plan or the best
// data-parallel tiling, whichever the tile path takes (given its workspace).
double tile_path_cost_us(int m, int n, int k) {
  double c = 0.0;
  if (split_slices(1, m, n, k, kSplitWsMax, &c) > 1) return c;
  HybPlan h;
  if (k > 0 && k % kBK == 0) {
    hyb_plan(1, m, n, k, h, &c);
    return c;
  }
  // K not a multiple of the k-tile: data-parallel only
  const long long cu = bch::device_cu_count();
  double best = 0.0;
  for (const TileOpt& o : kTileOpts) {
    const long long T = (long long)((m + o.bm - 1) / o.bm) * ((n + o.bn - 1) / o.bn);
    const double t = (double)((T + cu - 1) / cu) * ((k + kBK - 1) / kBK) * 7.4 * o.bm * o.bn / 65536.0 / o.eff;
    if (best == 0.0 || t < best) best = t;
  }
  return best;
}

// ---- whole rounds of 256 x 256 tiles on part of C, the rest planned on its own (the mixed plan) ----
// The hybrid plan's split tiles and the smaller tiles it picks to fill the last round cost
// efficiency over the whole matrix.  Where the 256 x 256 tiles make at least one whole round,
// the mixed plan runs j whole rounds of them on the first rows (or columns) of C, data-parallel,
// then the remaining rows (or columns) as a call of their own (split-K, hybrid or
// data-parallel, as planned for that shape).  Same box, two runs each, TFLOP/s, against the
// plan for the whole matrix: 4096 x 11008 x 4096 138.9 -> 141.5 (columns 0..8191 first),
// 11008 x 4096 x 4096 139.2 -> 141.5 (rows 0..8191), 8192 x 11008 x 4096 140.2 -> 144.6,
// 3072 x 11008 x 4096 138.4 -> 140.0, 4096 x 14336 x 4096 143.3 -> 145.0; 5120^3 142.1 ->
// 138.7, which the model rejects.  Chosen when the model puts it 1% ahead of the whole-matrix
// plan; the split runs along rows or columns, with j from 1 to the whole rounds available.
// Only the first level splits: the rest is planned without the mixed plan.
// The second launch's fixed cost in the model: its prologue, the first launch's last C stores
// that nothing overlaps, and the gap between the launches.  At 16 us the model picks, among
// 26 shapes measured both ways (K 1024 and 4096), every one that gained (1.1-6.0%) at K 4096
// and leaves out the two that lost (6144 x 6144 x 1024 -2.9%, 4100 x 4100 x 1024 -1.2%); two
// it still takes at K 1024 measured within 0.4% either way.
constexpr double kMixFixedUs = 16.0;

struct MixPlan {
  int axis = -1;  // 0: rows [0, split) first; 1: columns [0, split) first
  int split = 0;
};

bool mix_plan(int batch, int m, int n, int k, MixPlan& out) {
  if (batch != 1 || k <= 0 || k % kBK != 0) return false;
  const long long cu = bch::device_cu_count();
  const int mt = (m + 255) / 256, nt = (n + 255) / 256;
  const long long rounds = (long long)mt * nt / cu;
  if (rounds < 1) return false;
  const double nk = k / kBK;
  double best = 0.99 * tile_path_cost_us(m, n, k);
  bool found = false;
  for (int axis = 0; axis < 2; ++axis) {
    const int along = axis == 0 ? mt : nt, across = axis == 0 ? nt : mt;
    for (long long j = rounds; j >= 1; --j) {
      const long long c = j * cu / across;  // whole tile rows (columns) that fit j rounds
      if (c < 1 || c >= along) continue;
      const int split = (int)(256 * c);
      const double first = (double)((c * across + cu - 1) / cu) * nk * 7.4;
      const double rest = axis == 0 ? tile_path_cost_us(m - split, n, k) : tile_path_cost_us(m, n - split, k);
      const double cost = first + rest + kMixFixedUs;
      if (cost < best) {
        best = cost;
        found = true;
        out.axis = axis;
        out.split = split;
      }
    }
  }
  return found;
}

// C[tile j's rows and columns] = act(sum over s < S of P[s][j] (+ bias)) for the r split
// tiles j (logical tiles tile0 + j, in the kernel's grouped order); V: four columns per
// thread (N % 4 == 0, ldc % 4 == 0, C and bias 16-byte aligned)
template <bool V, int BM, int BN>
__global__ __launch_bounds__(256) void sgemm_tail_reduce(int M, int N, int tiles_m, int tiles_n, int tile0, int r,
                                                         int S, const float* __restrict__ P, float* __restrict__ C,
                                                         int ldc, const float* __restrict__ bias, int act) {
  constexpr int TS = BM * BN;
  constexpr int w = V ? 4 : 1;
  const long long total = (long long)r * TS / w;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long e = i * w;
    const int j = (int)(e / TS), l = (int)(e - (long long)j * TS);
    const int lr = l / BN, lc = l - lr * BN;
    const int L = tile0 + j, group_size = 8 * tiles_n, g = L / group_size, first_m = g * 8;
    const int gm = min(tiles_m - first_m, 8), within = L - g * group_size;
    const int row = (first_m + within % gm) * BM + lr, col = (within / gm) * BN + lc;
    if (row >= M || col >= N) continue;
    const float* src = P + (long long)j * TS + l;
    if constexpr (V) {
      float4 acc = *reinterpret_cast<const float4*>(src);
      for (int s = 1; s < S; ++s) {
        const float4 x = *reinterpret_cast<const float4*>(src + (long long)s * r * TS);
        acc.x += x.x;
        acc.y += x.y;
        acc.z += x.z;
        acc.w += x.w;
      }
      if (bias) {
        acc.x += bias[col];
        acc.y += bias[col + 1];
        acc.z += bias[col + 2];
        acc.w += bias[col + 3];
      }
      acc = make_float4(bch::activate(acc.x, act), bch::activate(acc.y, act), bch::activate(acc.z, act),
                        bch::activate(acc.w, act));
      *reinterpret_cast<float4*>(C + (long long)row * ldc + col) = acc;
    } else {
      float acc = src[0];
      for (int s = 1; s < S; ++s) acc += src[(long long)s * r * TS];
      if (bias) acc += bias[col];
      C[(long long)row * ldc + col] = bch::activate(acc, act);
    }
  }
}

template <int BM, int BN>
hipError_t launch_tail_reduce(hipStream_t s, int m, int n, const HybPlan& h, const float* P, float* C, int ldc,
                              const float* bias, int act) {
  const int tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  const bool v = n % 4 == 0 && ldc % 4 == 0 && aligned16(C) && (bias == nullptr || aligned16(bias));
  const long long work = (long long)h.r * BM * BN / (v ? 4 : 1);
  const int blocks = (int)std::min<long long>((work + 255) / 256, 4096);
  if (v)
    hipLaunchKernelGGL((sgemm_tail_reduce<true, BM, BN>), dim3(blocks), dim3(256), 0, s, m, n, tm, tn, h.ndp, h.r,
                       h.S, P, C, ldc, bias, act);
  else
    hipLaunchKernelGGL((sgemm_tail_reduce<false, BM, BN>), dim3(blocks), dim3(256), 0, s, m, n, tm, tn, h.ndp, h.r,
                       h.S, P, C, ldc, bias, act);
  return hipGetLastError();
}

// mode 0: unguarded loads; mode 1: float4-guarded (K % 32 == 0 here, so the one-add form)
template <bool TB, bool EPI>
hipError_t launch_hyb(int mode, const HybPlan& h, hipStream_t s, int m, int n, int k, const float* A, int lda,
                      const float* B, int ldb, float* C, int ldc, const float* bias, int act, float* P) {
#define BCH_HYB(BM_, BN_)                                                                                         \
  (mode == 0 ? launch_hyb_tiles<BM_, BN_, kBK, false, TB, EPI, false, false>(s, m, n, k, A, lda, B, ldb, C, ldc,  \
                                                                            bias, act, h.ndp, h.r, h.S, h.kt, P) \
             : launch_hyb_tiles<BM_, BN_, kBK, true, TB, EPI, true, true>(s, m, n, k, A, lda, B, ldb, C, ldc, bias, \
                                                                         act, h.ndp, h.r, h.S, h.kt, P))
  hipError_t e = h.t == Tile::k256x256   ? BCH_HYB(256, 256)
                 : h.t == Tile::k256x128 ? BCH_HYB(256, 128)
                                         : BCH_HYB(128, 128);
#undef BCH_HYB
  if (e != hipSuccess) return e;
  return h.t == Tile::k256x256   ? launch_tail_reduce<256, 256>(s, m, n, h, P, C, ldc, bias, act)
         : h.t == Tile::k256x128 ? launch_tail_reduce<256, 128>(s, m, n, h, P, C, ldc, bias, act)
                                 : launch_tail_reduce<128, 128>(s, m, n, h, P, C, ldc, bias, act);
}

// [n][k] weights with 32 < m <= 64 and n >= 8192: two passes of the m <= 32 path.  Same box,
// two runs each, against the tile path (bias + ReLU): 33 / 48 / 64 x 11008 x 4096 99.5 / 100.9
// / 103.0 -> 70.7 / 76.0 / 83.0 us; at n = 4096 the tiles fill the CUs and stay ahead (48 x 4096
// x 4096 40.0 against 44.1 us, 64 x 4096 x 11008 91.5 against 93.6).
bool nt_two_pass(int m, int n, int k, const float* A, int lda, const float* B, int ldb) {
  return m > 32 && m <= 64 && n >= 8192 && bch::sgemm_skinny_nt_applies(32, n, k, A, lda, B, ldb);
}

}  // namespace

namespace bch {

static const char* tile_path_name(int m, int n, int k, bool allow_mix);

const char* sgemm_kernel_name(int m, int n, int k) {
  if (sgemm_skinny_applies(m, n, k, nullptr, k, nullptr, n)) return sgemm_skinny_kernel_name(m);
  return tile_path_name(m, n, k, true);
}

// The tile path's kernels for lda = k, ldb = n and 16-byte aligned operands.
static const char* tile_path_name(int m, int n, int k, bool allow_mix) {
  MixPlan mp;
  if (allow_mix && mix_plan(1, m, n, k, mp)) {
    const int m1 = mp.axis == 0 ? mp.split : m, n1 = mp.axis == 1 ? mp.split : n;
    const bool fast = m1 % 256 == 0 && n1 % 256 == 0 && n % 4 == 0;
    thread_local std::string name;
    name = std::string(fast ? "sgemm_mfma_kernel<256,256,32,false>" : "sgemm_mfma_kernel<256,256,32,true,v4>") +
           (mp.axis == 0 ? " rows then " : " columns then ") +
           (mp.axis == 0 ? tile_path_name(m - m1, n, k, false) : tile_path_name(m, n - n1, k, false));
    return name.c_str();
  }
  if (small_tile_plan(1, m, n, k)) return "sgemm_mfma_kernel<64,64,64,false>";
  const Tile t = pick_tile(1, m, n);
  // with lda = k and ldb = n, and 16-byte aligned operands
  const bool check = !(m % tile_m(t) == 0 && n % tile_n(t) == 0 && k % kBK == 0 && k % 4 == 0 && n % 4 == 0);
  const bool v4 = k >= 4 && k % 4 == 0 && n % 4 == 0;
  if (split_slices(1, m, n, k) > 1) {  // slices of 32-k tiles (k % 32 == 0)
    const bool fast = m % tile_m(t) == 0 && n % tile_n(t) == 0 && n % 4 == 0;
    static const char* const split_names[3][3] = {
        {"sgemm_mfma_kernel<256,256,32,false>+sgemm_splitk_reduce", "sgemm_mfma_kernel<256,256,32,true,v4>+sgemm_splitk_reduce",
         "sgemm_mfma_kernel<256,256,32,true>+sgemm_splitk_reduce"},
        {"sgemm_mfma_kernel<256,128,32,false>+sgemm_splitk_reduce", "sgemm_mfma_kernel<256,128,32,true,v4>+sgemm_splitk_reduce",
         "sgemm_mfma_kernel<256,128,32,true>+sgemm_splitk_reduce"},
        {"sgemm_mfma_kernel<128,128,32,false>+sgemm_splitk_reduce", "sgemm_mfma_kernel<128,128,32,true,v4>+sgemm_splitk_reduce",
         "sgemm_mfma_kernel<128,128,32,true>+sgemm_splitk_reduce"}};
    return split_names[static_cast<int>(t)][fast ? 0 : v4 ? 1 : 2];
  }
  HybPlan h;
  if (hyb_plan(1, m, n, k, h)) {
    const bool fast = m % tile_m(h.t) == 0 && n % tile_n(h.t) == 0 && n % 4 == 0;
    static const char* const hyb_names[3][2] = {
        {"sgemm_mfma_kernel<256,256,32,false,hyb>+sgemm_tail_reduce", "sgemm_mfma_kernel<256,256,32,true,v4,hyb>+sgemm_tail_reduce"},
        {"sgemm_mfma_kernel<256,128,32,false,hyb>+sgemm_tail_reduce", "sgemm_mfma_kernel<256,128,32,true,v4,hyb>+sgemm_tail_reduce"},
        {"sgemm_mfma_kernel<128,128,32,false,hyb>+sgemm_tail_reduce", "sgemm_mfma_kernel<128,128,32,true,v4,hyb>+sgemm_tail_reduce"}};
    if (fast || v4) return hyb_names[static_cast<int>(h.t)][fast ? 0 : 1];
  }
  return tile_name(t, !check ? 0 : v4 ? 1 : 2);
}

// The tile path's scratch: split-K partials, or the hybrid plan's.  `optional` false: the
// plan within bch_sgemm_noalloc's 16 MiB (fewer split slices, no hybrid plan).
static size_t tile_workspace_bytes(int batch, int m, int n, int k, bool optional, bool allow_mix = true) {
  MixPlan mp;
  if (allow_mix && mix_plan(batch, m, n, k, mp))  // the whole tiles need none; the rest is a call of its own
    return mp.axis == 0 ? tile_workspace_bytes(1, m - mp.split, n, k, optional, false)
                        : tile_workspace_bytes(1, m, n - mp.split, k, optional, false);
  const int sl = split_slices(batch, m, n, k, optional ? kSplitWsMax : kSplitWsSmall);
  if (sl > 1) return (size_t)sl * batch * m * n * sizeof(float);
  HybPlan h;
  return optional && hyb_plan(batch, m, n, k, h) ? hyb_bytes(h) : 0;
}

size_t sgemm_workspace_bytes(int batch, int m, int n, int k) {
  if (batch == 1 && sgemm_skinny_applies(m, n, k, nullptr, k, nullptr, n))
    return sgemm_skinny_workspace_bytes(m, n, k);
  return tile_workspace_bytes(batch, m, n, k, true);
}

size_t sgemm_required_workspace_bytes(int batch, int m, int n, int k) {
  // 32 < m <= 64 takes the tile path where the skinny partials exceed the small scratch
  if (batch == 1 && sgemm_skinny_applies(m, n, k, nullptr, k, nullptr, n) &&
      (m <= 32 || sgemm_skinny_workspace_bytes(m, n, k) <= kSplitWsSmall))
    return sgemm_skinny_workspace_bytes(m, n, k);
  return tile_workspace_bytes(batch, m, n, k, false);
}

size_t sgemm_ex_workspace_bytes(bool transb, int batch, int m, int n, int k, int lda, int ldb) {
  if (!transb) return sgemm_workspace_bytes(batch, m, n, k);
  if (batch == 1 && sgemm_skinny_nt_applies(m, n, k, nullptr, lda, nullptr, ldb))
    return sgemm_skinny_nt_workspace_bytes(m, n, k);
  if (batch == 1 && nt_two_pass(m, n, k, nullptr, lda, nullptr, ldb))
    return std::max(sgemm_skinny_nt_workspace_bytes(32, n, k), sgemm_skinny_nt_workspace_bytes(m - 32, n, k));
  return tile_workspace_bytes(batch, m, n, k, true);
}

hipError_t launch_sgemm(hipStream_t s, int batch, int m, int n, int k, const float* A, int lda, long long sA,
                        const float* B, int ldb, long long sB, float* C, int ldc, long long sC, void* ws,
                        size_t ws_bytes) {
  return launch_sgemm_ex(s, false, batch, m, n, k, A, lda, sA, B, ldb, sB, nullptr, 0, C, ldc, sC, ws, ws_bytes);
}

}  // namespace bch

namespace {

// The tile path of launch_sgemm_ex: split-K, the mixed plan (allow_mix), the hybrid plan or the
// data-parallel tiling.
hipError_t launch_tile_path(hipStream_t s, bool transb, int batch, int m, int n, int k, const float* A, int lda,
                            long long sA, const float* B, int ldb, long long sB, const float* bias, int act,
                            float* C, int ldc, long long sC, void* ws, size_t ws_bytes, bool allow_mix);

}  // namespace

namespace bch {

hipError_t launch_sgemm_ex(hipStream_t s, bool transb, int batch, int m, int n, int k, const float* A, int lda,
                           long long sA, const float* B, int ldb, long long sB, const float* bias, int act,
                           float* C, int ldc, long long sC, void* ws, size_t ws_bytes) {
  if (batch <= 0 || m <= 0 || n <= 0) return hipSuccess;
  // m <= 32: the skinny kernels always (their partials sized by the caller); 32 < m <= 64:
  // the 64-row skinny kernel when its partials fit the scratch at hand, else the tiles
  if (!transb && batch == 1 && sgemm_skinny_applies(m, n, k, A, lda, B, ldb) &&
      (m <= 32 || (ws != nullptr && ws_bytes >= sgemm_skinny_workspace_bytes(m, n, k))))
    return launch_sgemm_skinny(s, m, n, k, A, lda, B, ldb, C, ldc, ws, ws_bytes, bias, act);
  if (transb && batch == 1 && sgemm_skinny_nt_applies(m, n, k, A, lda, B, ldb))
    return launch_sgemm_skinny_nt(s, m, n, k, A, lda, B, ldb, C, ldc, ws, ws_bytes, bias, act);
  // 32 < m <= 64 with [n][k] weights: the 32-row kernels twice, on rows 0..31 and 32..m-1 (the
  // second pass streams the weights again, largely from the Infinity Cache)
  if (transb && batch == 1 && nt_two_pass(m, n, k, A, lda, B, ldb)) {
    hipError_t e = launch_sgemm_skinny_nt(s, 32, n, k, A, lda, B, ldb, C, ldc, ws, ws_bytes, bias, act);
    if (e != hipSuccess) return e;
    return launch_sgemm_skinny_nt(s, m - 32, n, k, A + 32LL * lda, lda, B, ldb, C + 32LL * ldc, ldc, ws, ws_bytes,
                                  bias, act);
  }
  return launch_tile_path(s, transb, batch, m, n, k, A, lda, sA, B, ldb, sB, bias, act, C, ldc, sC, ws, ws_bytes,
                          true);
}

}  // namespace bch

namespace {

hipError_t launch_tile_path(hipStream_t s, bool transb, int batch, int m, int n, int k, const float* A, int lda,
                            long long sA, const float* B, int ldb, long long sB, const float* bias, int act,
                            float* C, int ldc, long long sC, void* ws, size_t ws_bytes, bool allow_mix) {
  if (small_tile_ok(batch, m, n, k, A, lda, sA, B, ldb, sB)) {
    const bool epi = bias != nullptr || act != 0;
#define BCH_SMALL(TB_, EPI_)                                                                                       \
  launch_tiles<64, 64, kSmallBK, false, TB_, EPI_>(s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act)
    return transb ? (epi ? BCH_SMALL(true, true) : BCH_SMALL(true, false))
                  : (epi ? BCH_SMALL(false, true) : BCH_SMALL(false, false));
#undef BCH_SMALL
  }
  const Tile t = pick_tile(batch, m, n);
  int sl = split_slices(batch, m, n, k);
  const size_t pbytes = (size_t)batch * m * n * sizeof(float);  // one slice's partials, every batch
  if (sl > 1 && (ws == nullptr || ws_bytes < (size_t)sl * pbytes))
    sl = ws == nullptr ? 1 : split_slices(batch, m, n, k, ws_bytes);  // fewer slices within the scratch at hand
  if (sl > 1 && ws != nullptr && ws_bytes >= (size_t)sl * pbytes) {
    // batch b, slice j (grid.z): A + b sA + j kc, B + b sB + j kc rows (columns for [n][k]),
    // into P[b][j] (m x n)
    const int kc = k / sl;
    float* P = static_cast<float*>(ws);
    const long long per = (long long)m * n;
    ZSplit z;
    z.nz = sl;
    z.sA = kc;
    z.sB = transb ? (long long)kc : (long long)kc * ldb;
    z.sC = per;
    // the slice offsets (kc a multiple of 32, times ldb) keep the batch strides' alignment
    const int mode = fast_ok(t, m, n, kc, A, lda, sA, B, ldb, sB)               ? 0
                     : vec4_ok(transb, m, n, kc, A, lda, sA, B, ldb, sB) ? 1
                                                                           : 2;
    hipError_t e = transb ? launch_tile_any<true, false>(mode, t, s, batch, m, n, kc, A, lda, sA, B, ldb, sB, P, n,
                                                         sl * per, nullptr, 0, z)
                          : launch_tile_any<false, false>(mode, t, s, batch, m, n, kc, A, lda, sA, B, ldb, sB, P, n,
                                                          sl * per, nullptr, 0, z);
    if (e != hipSuccess) return e;
    const bool v = n % 4 == 0 && ldc % 4 == 0 && aligned16(C) && (batch == 1 || sC % 4 == 0) &&
                   (bias == nullptr || aligned16(bias));
    const long long work = per * batch / (v ? 4 : 1);
    const int blocks = (int)std::min<long long>((work + 255) / 256, 4096);
    if (v)
      hipLaunchKernelGGL(sgemm_splitk_reduce<true>, dim3(blocks), dim3(256), 0, s, m, n, sl, batch, P, C, ldc, sC,
                         bias, act);
    else
      hipLaunchKernelGGL(sgemm_splitk_reduce<false>, dim3(blocks), dim3(256), 0, s, m, n, sl, batch, P, C, ldc, sC,
                         bias, act);
    return hipGetLastError();
  }
  const bool epi = bias != nullptr || act != 0;
  MixPlan mp;
  if (allow_mix && mix_plan(batch, m, n, k, mp)) {
    // whole rounds of 256 x 256 tiles on the first rows (columns) of C, then the rest as a call
    // of its own; the offsets are multiples of 256 rows (columns), which keeps the alignment
    const int m1 = mp.axis == 0 ? mp.split : m, n1 = mp.axis == 1 ? mp.split : n;
    const int mode1 = fast_ok(Tile::k256x256, m1, n1, k, A, lda, sA, B, ldb, sB)      ? 0
                      : vec4_ok(transb, m1, n1, k, A, lda, sA, B, ldb, sB) ? 1
                                                                             : 2;
    hipError_t e =
        transb ? (epi ? launch_tile_any<true, true>(mode1, Tile::k256x256, s, 1, m1, n1, k, A, lda, sA, B, ldb, sB, C,
                                                    ldc, sC, bias, act)
                      : launch_tile_any<true, false>(mode1, Tile::k256x256, s, 1, m1, n1, k, A, lda, sA, B, ldb, sB,
                                                     C, ldc, sC, bias, act))
               : (epi ? launch_tile_any<false, true>(mode1, Tile::k256x256, s, 1, m1, n1, k, A, lda, sA, B, ldb, sB,
                                                     C, ldc, sC, bias, act)
                      : launch_tile_any<false, false>(mode1, Tile::k256x256, s, 1, m1, n1, k, A, lda, sA, B, ldb, sB,
                                                      C, ldc, sC, bias, act));
    if (e != hipSuccess) return e;
    if (mp.axis == 0)
      return launch_tile_path(s, transb, 1, m - m1, n, k, A + (long long)m1 * lda, lda, sA, B, ldb, sB, bias, act,
                              C + (long long)m1 * ldc, ldc, sC, ws, ws_bytes, false);
    const float* B2 = transb ? B + (long long)n1 * ldb : B + n1;
    return launch_tile_path(s, transb, 1, m, n - n1, k, A, lda, sA, B2, ldb, sB, bias ? bias + n1 : nullptr, act,
                            C + n1, ldc, sC, ws, ws_bytes, false);
  }
  HybPlan h;
  if (hyb_plan(batch, m, n, k, h) && ws != nullptr && ws_bytes >= hyb_bytes(h)) {
    const int hmode = fast_ok(h.t, m, n, k, A, lda, sA, B, ldb, sB)                ? 0
                      : vec4_ok(transb, m, n, k, A, lda, sA, B, ldb, sB)          ? 1
                                                                                   : 2;
    if (hmode != 2) {
      float* P = static_cast<float*>(ws);
      if (transb)
        return epi ? launch_hyb<true, true>(hmode, h, s, m, n, k, A, lda, B, ldb, C, ldc, bias, act, P)
                   : launch_hyb<true, false>(hmode, h, s, m, n, k, A, lda, B, ldb, C, ldc, bias, act, P);
      return epi ? launch_hyb<false, true>(hmode, h, s, m, n, k, A, lda, B, ldb, C, ldc, bias, act, P)
                 : launch_hyb<false, false>(hmode, h, s, m, n, k, A, lda, B, ldb, C, ldc, bias, act, P);
    }
  }
  // the [n][k] tile loads need the same alignment as the [k][n] ones (ldb, sB multiples of 4); a
  // [n][k] B needs only K % 4 == 0 for whole float4, but N % 4 is kept for one rule
  const int mode = fast_ok(t, m, n, k, A, lda, sA, B, ldb, sB) ? 0
                   : vec4_ok(transb, m, n, k, A, lda, sA, B, ldb, sB) ? 1
                                                                 : 2;
  if (transb)
    return epi ? launch_tile_any<true, true>(mode, t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act)
               : launch_tile_any<true, false>(mode, t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias,
                                              act);
  return epi ? launch_tile_any<false, true>(mode, t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act)
             : launch_tile_any<false, false>(mode, t, s, batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC, bias,
                                             act);
}

}  // namespace
