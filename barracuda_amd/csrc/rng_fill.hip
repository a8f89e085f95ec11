// rng_fill.hip -- the reference's seeded generators, filled on the device.
//
// Restates crates/barracuda/src/rng.rs:20-70 (Knuth LCG, increment 1,
// u = (state >> 11) * 2^-53) and crates/barracuda/src/ops/lattice/
// constants.rs:11-49 (MMIX increment, Box-Muller with u1 guarded by 1e-30,
// cos branch) so that synthetic inputs of any size are produced in HBM,
// element-for-element identical to a sequential host fill in argument
// order.  Each thread jumps ahead to its first element with the affine map
// x -> a^n x + c (a^n - 1)/(a - 1) (mod 2^64), computed by squaring, then
// steps sequentially through a contiguous chunk.
#include "bch_internal.h"

#include <stdint.h>

namespace {

constexpr uint64_t kMul = 6364136223846793005ULL;
constexpr int kChunk = 16;

__host__ __device__ inline void lcg_jump(uint64_t inc, uint64_t n, uint64_t& A, uint64_t& Cc) {
  uint64_t acc_a = 1, acc_c = 0, cur_a = kMul, cur_c = inc;
  while (n) {
    if (n & 1) {
      acc_c = cur_a * acc_c + cur_c;
      acc_a = cur_a * acc_a;
    }
    cur_c = cur_a * cur_c + cur_c;
    cur_a = cur_a * cur_a;
    n >>= 1;
  }
  A = acc_a;
  Cc = acc_c;
}

__device__ inline double to_unit(uint64_t s) { return (double)(s >> 11) * (1.0 / 9007199254740992.0); }

__global__ __launch_bounds__(256) void fill_uniform_kernel(float* __restrict__ out, uint64_t n,
                                                           uint64_t state, double lo, double span) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t i0 = t * kChunk;
  if (i0 >= n) return;
  uint64_t a, c;
  lcg_jump(1, i0, a, c);
  uint64_t s = a * state + c;
  const uint64_t end = i0 + kChunk < n ? i0 + kChunk : n;
  for (uint64_t i = i0; i < end; ++i) {
    s = s * kMul + 1;
    out[i] = (float)(lo + span * to_unit(s));
  }
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float* __restrict__ out, uint64_t n,
                                                          uint64_t state, uint64_t inc, double mu,
                                                          double sigma) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t i0 = t * kChunk;
  if (i0 >= n) return;
  uint64_t a, c;
  lcg_jump(inc, 2 * i0, a, c);
  uint64_t s = a * state + c;
  const uint64_t end = i0 + kChunk < n ? i0 + kChunk : n;
  const double two_pi = 6.283185307179586476925286766559;
  for (uint64_t i = i0; i < end; ++i) {
    s = s * kMul + inc;
    const double u1 = to_unit(s);
    s = s * kMul + inc;
    const double u2 = to_unit(s);
    const double g = sqrt(-2.0 * log(u1 > 1e-30 ? u1 : 1e-30)) * cos(two_pi * u2);
    out[i] = (float)(mu + sigma * g);
  }
}

}  // namespace

namespace bch {

constexpr uint64_t kIncMmix = 1442695040888963407ULL;

uint64_t lcg_advance(uint64_t state, uint64_t inc, uint64_t n) {
  uint64_t a, c;
  lcg_jump(inc, n, a, c);
  return a * state + c;
}

hipError_t launch_fill_uniform(hipStream_t s, float* out, uint64_t n, uint64_t state, double lo,
                               double hi) {
  if (n == 0) return hipSuccess;
  const uint64_t threads = (n + kChunk - 1) / kChunk;
  const uint64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffULL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fill_uniform_kernel, dim3((unsigned)blocks), dim3(256), 0, s, out, n, state, lo,
                     hi - lo);
  return hipGetLastError();
}

hipError_t launch_fill_normal(hipStream_t s, float* out, uint64_t n, uint64_t state, double mu,
                              double sigma) {
  if (n == 0) return hipSuccess;
  const uint64_t threads = (n + kChunk - 1) / kChunk;
  const uint64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffULL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, s, out, n, state,
                     kIncMmix, mu, sigma);
  return hipGetLastError();
}

}  // namespace bch
