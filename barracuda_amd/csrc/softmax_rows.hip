// softmax_rows.hip -- row-wise f32 softmax for gfx950.
//
// Replaces the reference's row softmax paths: Tensor::softmax_dim
// (crates/barracuda/src/ops/tensor_axis_ops.rs:67-126, host f32 loops) and
// the attention row softmax K7 (shaders/activation/attention_softmax_f64.wgsl
// :24-58, one thread per row, five sweeps).  Same contract: y = exp(x - max)
// / sum over each row, max-subtracted.
//
// Design (HBM-bound: one read + one write of the matrix is the floor):
//   * rows with cols % 4 == 0 and cols <= 4096: one wavefront per row; the
//     row is loaded once with 128-bit coalesced loads (lane l takes float4
//     l, l+64, ...) and stays in registers; max and sum are wavefront
//     all-reductions built from DPP row operations plus four v_readlane
//     across the 16-lane rows; the output is written once.
//   * anything else: one workgroup per row, an online (max, sum) pass and a
//     second read that writes; scalar loads, any cols.
//   * axis != last: one thread per (outer, inner) slice, coalesced across
//     inner, online (max, sum) then a writing pass.
// exp(x) is 2^(x log2 e) on v_exp_f32 with the product's rounding error
// carried as a first-order correction (x*log2e split into p + e exactly with
// one fma), which keeps it within ~2 ulp of a correctly rounded expf over
// the range softmax feeds it (x - max <= 0); exp(-inf) = 0.
#include "bch_internal.h"

#include <math.h>

namespace {

constexpr float kLog2E = 1.44269502162933349609375f;     // float(log2 e)
constexpr float kLog2ELo = 1.925963033500011829e-8f;      // log2 e - kLog2E
constexpr float kLn2 = 0.693147180559945309f;

__device__ __forceinline__ float exp_f32(float x) {
  // exp(x) == 0 in f32 below -110 (2^-158 < the smallest subnormal); the
  // clamp also keeps -inf out of the fma split below (-inf + inf = NaN).
  // NaN fails the comparison and propagates.
  x = x < -110.0f ? -110.0f : x;
  float p = x * kLog2E;
  float e = fmaf(x, kLog2E, -p);  // exact rounding error of x*kLog2E
  e = fmaf(x, kLog2ELo, e);
  float r = __builtin_amdgcn_exp2f(p);
  return fmaf(r, e * kLn2, r);    // 2^p * (1 + e ln 2)
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, true));
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

struct OpMax {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpSum {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// All-reduce over the 64 lanes of a wavefront; every lane gets the result.
//   quad_perm[1,0,3,2] (0xB1): lane ^ 1      quad_perm[2,3,0,1] (0x4E): lane ^ 2
//   row_half_mirror (0x141): lane i <-> 7-i within 8, joins the two quads
//   row_mirror      (0x140): lane i <-> 15-i within 16, joins the two halves
// then the four 16-lane rows are combined through v_readlane (uniform).
template <typename Op>
__device__ __forceinline__ float wave_allreduce(float v, Op op) {
  v = op(v, dpp<0xB1>(v));
  v = op(v, dpp<0x4E>(v));
  v = op(v, dpp<0x141>(v));
  v = op(v, dpp<0x140>(v));
  float r0 = readlane(v, 0), r1 = readlane(v, 16);
  float r2 = readlane(v, 32), r3 = readlane(v, 48);
  return op(op(r0, r1), op(r2, r3));
}

// One wavefront per row, NV float4 per lane (cols <= 256 * NV, cols % 4 == 0).
template <int NV>
__device__ __forceinline__ void softmax_rows_wave_body(
    const float* __restrict__ in, float* __restrict__ out, long long rows,
    int cols) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int nvec = cols >> 2;
  const float4* src = reinterpret_cast<const float4*>(in + row * (long long)cols);
  float4* dst = reinterpret_cast<float4*>(out + row * (long long)cols);
  float4 v[NV];
  const float ninf = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int idx = i * 64 + lane;
    v[i] = idx < nvec ? bch::load_nt(src + idx)
                      : make_float4(ninf, ninf, ninf, ninf);
  }
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
  mx = wave_allreduce(mx, OpMax());
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i * 64 + lane < nvec) {
      v[i].x = exp_f32(v[i].x - mx);
      v[i].y = exp_f32(v[i].y - mx);
      v[i].z = exp_f32(v[i].z - mx);
      v[i].w = exp_f32(v[i].w - mx);
      s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
  }
  s = wave_allreduce(s, OpSum());
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int idx = i * 64 + lane;
    if (idx < nvec) {
      float4 r = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
      bch::store_nt(r, dst + idx);
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void softmax_rows_wave(
    const float* __restrict__ in, float* __restrict__ out, long long rows,
    int cols) {
  softmax_rows_wave_body<NV>(in, out, rows, cols);
}

// Online update of (max m, sum s) with one element v; -inf contributes 0.
__device__ __forceinline__ void online_push(float& m, float& s, float v) {
  if (v > m) {
    s = s * exp_f32(m - v) + 1.0f;
    m = v;
  } else if (v != -INFINITY) {
    s += exp_f32(v - m);
  }
}

// Merge two online-softmax partial states (max m, sum of exp(x - m)).
__device__ __forceinline__ void merge_state(float& m, float& s, float m2, float s2) {
  float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  s = s * exp_f32(m - mn) + s2 * exp_f32(m2 - mn);
  m = mn;
}

// One workgroup (256 threads) per row, any cols.
__global__ __launch_bounds__(256) void softmax_rows_block(
    const float* __restrict__ in, float* __restrict__ out, long long rows,
    long long cols) {
  __shared__ float sm[4], ss[4];
  const long long row = blockIdx.x;
  const float* x = in + row * cols;
  float* y = out + row * cols;
  float m = -INFINITY, s = 0.0f;
  for (long long j = threadIdx.x; j < cols; j += 256) online_push(m, s, x[j]);
  // wave-level merge: all-reduce the max, rescale, all-reduce the sum
  float wm = wave_allreduce(m, OpMax());
  float ws = wave_allreduce(m == -INFINITY ? 0.0f : s * exp_f32(m - wm), OpSum());
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = wm;
    ss[w] = ws;
  }
  __syncthreads();
  float M = sm[0], S = ss[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) merge_state(M, S, sm[i], ss[i]);
  const float inv = 1.0f / S;
  for (long long j = threadIdx.x; j < cols; j += 256) y[j] = exp_f32(x[j] - M) * inv;
}

// Softmax along the middle axis of [outer, axis, inner], thread per slice.
__global__ __launch_bounds__(256) void softmax_axis_strided(
    const float* __restrict__ in, float* __restrict__ out, long long outer,
    long long axis, long long inner) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const long long o = t / inner, i = t % inner;
  const float* x = in + o * axis * inner + i;
  float* y = out + o * axis * inner + i;
  float m = -INFINITY, s = 0.0f;
  for (long long j = 0; j < axis; ++j) online_push(m, s, x[j * inner]);
  const float inv = 1.0f / s;
  for (long long j = 0; j < axis; ++j) y[j * inner] = exp_f32(x[j * inner] - m) * inv;
}

int pick_nv(long long cols) {
  if (cols <= 256) return 1;
  if (cols <= 512) return 2;
  if (cols <= 1024) return 4;
  if (cols <= 2048) return 8;
  if (cols <= 4096) return 16;
  return 0;
}

bool wave_path(long long cols, const float* in, const float* out) {
  return (cols % 4) == 0 && pick_nv(cols) > 0 &&
         (reinterpret_cast<uintptr_t>(in) % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(out) % 16) == 0;
}

}  // namespace

namespace bch {

const char* softmax_kernel_name(long long rows, long long cols) {
  if ((cols % 4) == 0) {
    switch (pick_nv(cols)) {
      case 1: return "softmax_rows_wave<1>";
      case 2: return "softmax_rows_wave<2>";
      case 4: return "softmax_rows_wave<4>";
      case 8: return "softmax_rows_wave<8>";
      case 16: return "softmax_rows_wave<16>";
      default: break;
    }
  }
  return "softmax_rows_block";
}

hipError_t launch_softmax_rows(hipStream_t s, long long rows, long long cols,
                               const float* in, float* out) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (wave_path(cols, in, out)) {
    const long long blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks), block(256);
    switch (pick_nv(cols)) {
      case 1: hipLaunchKernelGGL(softmax_rows_wave<1>, grid, block, 0, s, in, out, rows, (int)cols); break;
      case 2: hipLaunchKernelGGL(softmax_rows_wave<2>, grid, block, 0, s, in, out, rows, (int)cols); break;
      case 4: hipLaunchKernelGGL(softmax_rows_wave<4>, grid, block, 0, s, in, out, rows, (int)cols); break;
      case 8: hipLaunchKernelGGL(softmax_rows_wave<8>, grid, block, 0, s, in, out, rows, (int)cols); break;
      default: hipLaunchKernelGGL(softmax_rows_wave<16>, grid, block, 0, s, in, out, rows, (int)cols); break;
    }
  } else {
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(softmax_rows_block, dim3((unsigned)rows), dim3(256), 0, s, in, out, rows, cols);
  }
  return hipGetLastError();
}

hipError_t launch_softmax_axis(hipStream_t s, long long outer, long long axis,
                               long long inner, const float* in, float* out) {
  if (outer <= 0 || axis <= 0 || inner <= 0) return hipSuccess;
  if (inner == 1) return launch_softmax_rows(s, outer, axis, in, out);
  const long long slices = outer * inner;
  const long long blocks = (slices + 255) / 256;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(softmax_axis_strided, dim3((unsigned)blocks), dim3(256), 0, s, in, out, outer, axis, inner);
  return hipGetLastError();
}

}  // namespace bch

// Unmangled entry for the code-object path (bch_launch_code_object): the
// cols == 2048 register-resident row softmax, 4 rows per 256-thread block.
extern "C" __global__ __launch_bounds__(256) void bch_softmax_rows_2048(
    const float* __restrict__ in, float* __restrict__ out, long long rows) {
  softmax_rows_wave_body<8>(in, out, rows, 2048);
}
