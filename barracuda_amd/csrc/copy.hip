// copy.hip -- device-to-device copy (bch_copy).
//
// A streaming copy: each wavefront owns one contiguous run of 256 float4
// (4 KB), lane l taking float4 l, l + 64, l + 128, l + 192 with all four
// loads in flight before the stores, as the element-wise kernels do; copies
// of 64 MB or more use non-temporal loads and stores.  Pointers or sizes that
// are not 16-byte multiples take a byte loop.  Besides duplicating buffers it
// is the reference kernel of known traffic (reads N bytes, writes N bytes)
// used to calibrate the HBM byte counters that profile the hot-path kernels.
// Measured (512 MiB copy, one box): a grid-stride loop over 8192 workgroups
// 192 us (5.6 TB/s); this layout 169.5 us (6.33 TB/s, 79% of 8 TB/s).
#include "bch_internal.h"

#include <stdint.h>

namespace {

constexpr int kRun = 4;  // float4 per lane of a wave's run

// Wave w of the grid copies float4 [256 w, 256 w + 256) of the n4 pieces.
template <bool NT>
__global__ __launch_bounds__(256) void copy_f4_kernel(float4* __restrict__ dst, const float4* __restrict__ src,
                                                      uint64_t n4) {
  const uint64_t base = ((uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 * kRun) + (threadIdx.x & 63);
  float4 v[kRun];
#pragma unroll
  for (int u = 0; u < kRun; ++u) {
    const uint64_t i = base + u * 64;
    if (i < n4) v[u] = NT ? bch::load_nt(src + i) : src[i];
  }
#pragma unroll
  for (int u = 0; u < kRun; ++u) {
    const uint64_t i = base + u * 64;
    if (i < n4) {
      if (NT)
        bch::store_nt(v[u], dst + i);
      else
        dst[i] = v[u];
    }
  }
}

__global__ __launch_bounds__(256) void copy_bytes_kernel(unsigned char* __restrict__ dst,
                                                         const unsigned char* __restrict__ src,
                                                         uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

namespace bch {

hipError_t launch_copy(hipStream_t s, void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes) & 15) == 0;
  const uint64_t n4 = bytes / 16;
  const uint64_t runs = (n4 + 1023) / 1024;  // workgroups of four 4 KB runs
  if (vec && runs <= 0x7fffffffULL) {
    if (bytes >= ((size_t)64 << 20))
      hipLaunchKernelGGL(copy_f4_kernel<true>, dim3((unsigned)runs), dim3(256), 0, s, static_cast<float4*>(dst),
                         static_cast<const float4*>(src), n4);
    else
      hipLaunchKernelGGL(copy_f4_kernel<false>, dim3((unsigned)runs), dim3(256), 0, s, static_cast<float4*>(dst),
                         static_cast<const float4*>(src), n4);
    return hipGetLastError();
  }
  uint64_t blocks = (bytes + 255) / 256;
  if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32 blocks per CU
  hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<unsigned char*>(dst),
                     static_cast<const unsigned char*>(src), (uint64_t)bytes);
  return hipGetLastError();
}

}  // namespace bch
