// softmax_f64.hip -- f64 row softmax for gfx950.
//
// The step between the two products of the ml.attention handler
// (crates/barracuda-core/src/ipc/methods/ml/forward.rs:130-140; its products
// Q K^T and P V run on bch_dgemm).  Per row of `cols` values:
//   m   = max_j x_j, folded from -inf with f64::max (NaN entries skipped)
//   e_j = exp(x_j - m)
//   y_j = e_j / sum_j e_j
// HBM-bound: one read and one write of the matrix (16 bytes per element).
//   * cols <= 2048: the row stays in registers, at most 8 doubles per lane
//     (occupancy 8): one wavefront per row up to 512 columns (four rows per
//     256-thread workgroup), the workgroup's four wavefronts per row up to
//     2048 (each a contiguous quarter; their max and sum combined through
//     LDS).  16-byte loads when cols is even and both matrices are 16-byte
//     aligned, 8-byte loads otherwise; wavefront all-reductions (DPP row ops
//     + v_readlane on both halves of each double); non-temporal loads and
//     stores (the matrix is streamed once).  Measured at 32768 x 2048 f64:
//     one wavefront per row with the row's 32 doubles per lane (occupancy 4)
//     5.1 TB/s, non-temporal 5.6 TB/s, two wavefronts per row 5.8-6.1 TB/s,
//     four 6.1-6.4 TB/s.
//   * 2048 < cols <= 8192: the same kernel with the workgroup's four
//     wavefronts per row and up to 32 doubles per lane (occupancy 4).
//   * longer rows: one 256-thread workgroup per row, three sweeps (max; sum
//     of exp; write), the second and third reading the row again from cache.
// in may equal out: every value is read before any value of its row is
// written (the register paths hold the row; the block path's last sweep
// starts after a barrier that follows the second sweep's reads, and each
// thread then reads only the elements it writes).
#include "bch_internal.h"

#include <math.h>

namespace {

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, true);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// fmax returns the other operand when one is NaN, as f64::max does.
struct MaxD {
  __device__ double operator()(double a, double b) const { return fmax(a, b); }
};
struct SumD {
  __device__ double operator()(double a, double b) const { return a + b; }
};

// All-reduce over the 64 lanes of a wavefront (the DPP sequence of
// bch::wave_allreduce, applied to both 32-bit halves).
template <typename Op>
__device__ __forceinline__ double wave_allreduce_f64(double v, Op op) {
  v = op(v, dpp_f64<0xB1>(v));
  v = op(v, dpp_f64<0x4E>(v));
  v = op(v, dpp_f64<0x141>(v));
  v = op(v, dpp_f64<0x140>(v));
  const double r0 = readlane_f64(v, 0), r1 = readlane_f64(v, 16);
  const double r2 = readlane_f64(v, 32), r3 = readlane_f64(v, 48);
  return op(op(r0, r1), op(r2, r3));
}

typedef double f64x2 __attribute__((ext_vector_type(2)));

// W wavefronts per row (W = 1: four rows per workgroup; W = 4: one).  Wave
// part p of a row holds its vectors p NV 64 + 64 i + lane (i < NV) of VEC
// doubles each; cols <= 64 W NV VEC.
template <int NV, int VEC, int W>
__global__ __launch_bounds__(256) void softmax_f64_rows(const double* in, double* out, long long rows, int cols) {
  static_assert(W == 1 || W == 4, "one or four wavefronts per row");
  __shared__ double sh[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long row = (long long)blockIdx.x * (4 / W) + wave / W;
  if (W == 1 && row >= rows) return;  // wave-uniform; with W = 4 the grid is exactly `rows`
  const int part = wave % W;
  const double* x = in + row * cols;
  double* y = out + row * cols;
  const int nvec = cols / VEC, base = part * NV * 64;
  double v[NV][VEC];
  double m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = base + i * 64 + lane;
    if (idx < nvec) {
      if constexpr (VEC == 2) {
        const f64x2 t = __builtin_nontemporal_load(reinterpret_cast<const f64x2*>(x) + idx);
        v[i][0] = t.x;
        v[i][1] = t.y;
      } else {
        v[i][0] = __builtin_nontemporal_load(x + idx);
      }
#pragma unroll
      for (int c = 0; c < VEC; ++c) m = fmax(m, v[i][c]);
    }
  }
  m = wave_allreduce_f64(m, MaxD());
  if constexpr (W > 1) {
    if (lane == 0) sh[0][wave] = m;
    __syncthreads();
    m = fmax(fmax(sh[0][0], sh[0][1]), fmax(sh[0][2], sh[0][3]));
  }
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (base + i * 64 + lane < nvec) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        v[i][c] = exp(v[i][c] - m);
        s += v[i][c];
      }
    }
  }
  s = wave_allreduce_f64(s, SumD());
  if constexpr (W > 1) {
    if (lane == 0) sh[1][wave] = s;
    __syncthreads();
    s = (sh[1][0] + sh[1][1]) + (sh[1][2] + sh[1][3]);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = base + i * 64 + lane;
    if (idx < nvec) {
      if constexpr (VEC == 2) {
        const f64x2 o = {v[i][0] / s, v[i][1] / s};
        __builtin_nontemporal_store(o, reinterpret_cast<f64x2*>(y) + idx);
      } else {
        __builtin_nontemporal_store(v[i][0] / s, y + idx);
      }
    }
  }
}

// All-reduce over the 256 threads of a workgroup; every thread gets it.
// Must be reached by all threads of the block.
template <typename Op>
__device__ __forceinline__ double block_allreduce_f64(double v, Op op, double* sh) {
  v = wave_allreduce_f64(v, op);
  __syncthreads();  // sh may still be read from the previous call
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return op(op(sh[0], sh[1]), op(sh[2], sh[3]));
}

__global__ __launch_bounds__(256) void softmax_f64_block(const double* in, double* out, long long cols) {
  __shared__ double sh[4];
  const long long row = blockIdx.x;
  const double* x = in + row * cols;
  double* y = out + row * cols;
  double m = -INFINITY;
  for (long long j = threadIdx.x; j < cols; j += 256) m = fmax(m, x[j]);
  m = block_allreduce_f64(m, MaxD(), sh);
  double s = 0.0;
  for (long long j = threadIdx.x; j < cols; j += 256) s += exp(x[j] - m);
  s = block_allreduce_f64(s, SumD(), sh);
  for (long long j = threadIdx.x; j < cols; j += 256) y[j] = exp(x[j] - m) / s;
}

struct RowPlan {
  int nv, vec, w;  // nv == 0: the three-sweep block kernel
};

// At most 8 doubles per lane up to 2048 columns (one wavefront per row up to
// 512, four up to 2048), then up to 32 doubles per lane on four wavefronts
// per row up to 8192 (occupancy 4 instead of a three-sweep block kernel).
RowPlan row_plan(long long cols, bool aligned16) {
  const int vec = aligned16 && cols % 2 == 0 ? 2 : 1;
  const int w = cols <= 512 ? 1 : 4;
  const int most = cols <= 2048 ? 8 : 32;
  for (int nv = 1; nv * vec <= most; nv *= 2)
    if (cols <= 64LL * w * nv * vec) return {nv, vec, w};
  return {0, vec, 1};
}

template <int VEC, int W>
hipError_t launch_rows(hipStream_t s, int nv, long long rows, int cols, const double* in, double* out) {
  const dim3 grid((unsigned)(W == 1 ? (rows + 3) / 4 : rows)), block(256);
  switch (nv) {
    case 1: hipLaunchKernelGGL((softmax_f64_rows<1, VEC, W>), grid, block, 0, s, in, out, rows, cols); break;
    case 2: hipLaunchKernelGGL((softmax_f64_rows<2, VEC, W>), grid, block, 0, s, in, out, rows, cols); break;
    case 4: hipLaunchKernelGGL((softmax_f64_rows<4, VEC, W>), grid, block, 0, s, in, out, rows, cols); break;
    case 8: hipLaunchKernelGGL((softmax_f64_rows<8, VEC, W>), grid, block, 0, s, in, out, rows, cols); break;
    case 16:
      if constexpr (W == 4) {
        hipLaunchKernelGGL((softmax_f64_rows<16, VEC, 4>), grid, block, 0, s, in, out, rows, cols);
        break;
      }
      return hipErrorInvalidValue;
    case 32:
      if constexpr (W == 4 && VEC == 1) {
        hipLaunchKernelGGL((softmax_f64_rows<32, 1, 4>), grid, block, 0, s, in, out, rows, cols);
        break;
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

namespace bch {

const char* softmax_f64_kernel_name(long long rows, long long cols, bool aligned16) {
  (void)rows;
  static const char* const names[2][2][6] = {
      {{"softmax_f64_rows<1,1,1>", "softmax_f64_rows<2,1,1>", "softmax_f64_rows<4,1,1>", "softmax_f64_rows<8,1,1>", "",
        ""},
       {"softmax_f64_rows<1,1,4>", "softmax_f64_rows<2,1,4>", "softmax_f64_rows<4,1,4>", "softmax_f64_rows<8,1,4>",
        "softmax_f64_rows<16,1,4>", "softmax_f64_rows<32,1,4>"}},
      {{"softmax_f64_rows<1,2,1>", "softmax_f64_rows<2,2,1>", "softmax_f64_rows<4,2,1>", "", "", ""},
       {"softmax_f64_rows<1,2,4>", "softmax_f64_rows<2,2,4>", "softmax_f64_rows<4,2,4>", "softmax_f64_rows<8,2,4>",
        "softmax_f64_rows<16,2,4>", ""}}};
  const RowPlan p = row_plan(cols, aligned16);
  if (p.nv == 0) return "softmax_f64_block";
  return names[p.vec - 1][p.w == 4][__builtin_ctz(p.nv)];
}

hipError_t launch_softmax_rows_f64(hipStream_t s, long long rows, long long cols, const double* in, double* out) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const RowPlan p = row_plan(cols, aligned16);
  // rows in launches of at most kRowsPerLaunch (grids below 2^32 threads); a
  // chunk starts a whole number of rows in (an even count of doubles where
  // the 16-byte path runs), so the alignment the plan was chosen for holds
  for (long long r0 = 0; r0 < rows; r0 += kRowsPerLaunch) {
    const long long n = rows - r0 < kRowsPerLaunch ? rows - r0 : kRowsPerLaunch;
    const double* x = in + r0 * cols;
    double* y = out + r0 * cols;
    hipError_t e;
    if (p.nv > 0) {
      const int c = (int)cols;
      if (p.vec == 2)
        e = p.w == 1 ? launch_rows<2, 1>(s, p.nv, n, c, x, y) : launch_rows<2, 4>(s, p.nv, n, c, x, y);
      else
        e = p.w == 1 ? launch_rows<1, 1>(s, p.nv, n, c, x, y) : launch_rows<1, 4>(s, p.nv, n, c, x, y);
    } else {
      hipLaunchKernelGGL(softmax_f64_block, dim3((unsigned)n), dim3(256), 0, s, x, y, cols);
      e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace bch
