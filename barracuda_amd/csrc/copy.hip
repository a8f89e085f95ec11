// copy.hip -- device-to-device copy (bch_copy).
//
// A plain streaming copy: 16-byte loads and stores when both pointers and the
// size allow, bytes otherwise.  Besides duplicating buffers it is the
// reference kernel of known traffic (reads N bytes, writes N bytes) used to
// calibrate the HBM byte counters that profile the hot-path kernels.
#include "bch_internal.h"

#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void copy_f4_kernel(float4* __restrict__ dst,
                                                      const float4* __restrict__ src, uint64_t n4) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
    bch::store_nt(bch::load_nt(src + i), dst + i);
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
  const uint64_t n = vec ? bytes / 16 : bytes;
  uint64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32 blocks per CU
  if (vec)
    hipLaunchKernelGGL(copy_f4_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<float4*>(dst),
                       static_cast<const float4*>(src), n);
  else
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<unsigned char*>(dst), static_cast<const unsigned char*>(src), n);
  return hipGetLastError();
}

}  // namespace bch
