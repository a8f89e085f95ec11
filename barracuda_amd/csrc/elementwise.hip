// elementwise.hip -- the session's element-wise ops for gfx950.
//
// Replaces the inline WGSL element-wise shaders of TensorSession
// (crates/barracuda/src/session/pipelines.rs:76-145: add, sub, mul, negate,
// fma, scale, one thread per element) and the activation shaders it binds
// (ops/relu.rs -> relu_f64.wgsl, ops/gelu_wgsl.rs -> gelu_f64.wgsl).  Same
// contract per element:
//   add a+b   sub a-b   mul a*b   negate -a   fma fma(a, b, c)
//   scale a*s   relu max(a, 0)   gelu 0.5 a (1 + tanh(0.7978845608 (a + 0.044715 a^3)))
//
// HBM-bound (8 to 16 bytes per element).  Each wavefront owns one
// contiguous run of 256 float4 (4 KB per operand): lane l takes float4
// l, l + 64, l + 128, l + 192, all loads in flight before the math, so
// every load instruction of a wave covers 1 KB of consecutive addresses.
// One run per wave, no loop.  Large tensors (>= 64 MB moved) use
// non-temporal loads and stores: they stream past the caches.  Measured on
// one MI355X, GELU over 2^27 elements: this layout 167 us (80% of 8 TB/s)
// against 260 us for a grid-stride loop of four 16-byte pieces per thread
// (a 1 KB piece per wave every 8 MB); 2 or 8 pieces per lane and
// temporal accesses were slower.  The unaligned head/tail and misaligned
// operands take a scalar loop.
#include "bch_internal.h"

namespace {

constexpr int kEwAdd = 0, kEwSub = 1, kEwMul = 2, kEwNeg = 3, kEwFma = 4, kEwScale = 5, kEwRelu = 6,
              kEwGelu = 7;

template <int OP>
__device__ __forceinline__ float ew(float a, float b, float c, float s) {
  if (OP == kEwAdd) return a + b;
  if (OP == kEwSub) return a - b;
  if (OP == kEwMul) return a * b;
  if (OP == kEwNeg) return -a;
  if (OP == kEwFma) return fmaf(a, b, c);
  if (OP == kEwScale) return a * s;
  if (OP == kEwRelu) return fmaxf(a, 0.0f);
  return bch::gelu_tanh(a);
}

// operands read by OP: a always, b for the binary ops and fma, c for fma
template <int OP>
constexpr bool uses_b() {
  return OP == kEwAdd || OP == kEwSub || OP == kEwMul || OP == kEwFma;
}

template <int OP>
__device__ __forceinline__ float4 ew4(float4 a, float4 b, float4 c, float s) {
  return make_float4(ew<OP>(a.x, b.x, c.x, s), ew<OP>(a.y, b.y, c.y, s), ew<OP>(a.z, b.z, c.z, s),
                     ew<OP>(a.w, b.w, c.w, s));
}

template <bool NT>
__device__ __forceinline__ float4 load4(const float4* p) {
  if (NT) return bch::load_nt(p);
  return *p;
}
template <bool NT>
__device__ __forceinline__ void store4(float4 v, float4* p) {
  if (NT)
    bch::store_nt(v, p);
  else
    *p = v;
}

constexpr int kRun = 4;  // float4 per lane of a wave's run

// Wave w of the grid covers float4 [256 w, 256 w + 256) of the n4 pieces.
template <int OP, bool NT>
__global__ __launch_bounds__(256) void ew_vec(long long n4, const float4* a, const float4* b, const float4* c,
                                              float s, float4* o) {
  const long long base = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 * kRun) + (threadIdx.x & 63);
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 va[kRun], vb[kRun], vc[kRun];
#pragma unroll
  for (int u = 0; u < kRun; ++u) {
    const long long i = base + u * 64;
    const bool in = i < n4;
    va[u] = in ? load4<NT>(a + i) : z;
    vb[u] = uses_b<OP>() && in ? load4<NT>(b + i) : z;
    vc[u] = OP == kEwFma && in ? load4<NT>(c + i) : z;
  }
#pragma unroll
  for (int u = 0; u < kRun; ++u) {
    const long long i = base + u * 64;
    if (i < n4) store4<NT>(ew4<OP>(va[u], vb[u], vc[u], s), o + i);
  }
}

template <int OP>
__global__ __launch_bounds__(256) void ew_scalar(long long begin, long long n, const float* a, const float* b,
                                                 const float* c, float s, float* o) {
  const long long stride = (long long)gridDim.x * 256;
  for (long long i = begin + (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    o[i] = ew<OP>(a[i], uses_b<OP>() ? b[i] : 0.0f, OP == kEwFma ? c[i] : 0.0f, s);
}

unsigned grid_for(long long work) {
  // a few workgroups per CU (256 CUs), never more than the work needs
  const long long want = (work + 255) / 256;
  return (unsigned)(want < 2048 ? (want < 1 ? 1 : want) : 2048);
}

constexpr long long kNtBytes = 64LL << 20;  // streams at least this large bypass the caches

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int OP>
hipError_t launch_op(hipStream_t st, long long n, const float* a, const float* b, const float* c, float s,
                     float* o) {
  bool vec = aligned16(a) && aligned16(o);
  if (uses_b<OP>()) vec = vec && aligned16(b);
  if (OP == kEwFma) vec = vec && aligned16(c);
  long long done = 0;
  if (vec && n >= 4) {
    const long long n4 = n / 4;
    const long long blocks = (n4 + 4 * 64 * kRun - 1) / (4 * 64 * kRun);
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    const int streams = 2 + (uses_b<OP>() ? 1 : 0) + (OP == kEwFma ? 1 : 0);
    const bool nt = (long long)streams * 4 * n >= kNtBytes;
    const float4 *a4 = reinterpret_cast<const float4*>(a), *b4 = reinterpret_cast<const float4*>(b),
                 *c4 = reinterpret_cast<const float4*>(c);
    float4* o4 = reinterpret_cast<float4*>(o);
    if (nt)
      hipLaunchKernelGGL((ew_vec<OP, true>), dim3((unsigned)blocks), dim3(256), 0, st, n4, a4, b4, c4, s, o4);
    else
      hipLaunchKernelGGL((ew_vec<OP, false>), dim3((unsigned)blocks), dim3(256), 0, st, n4, a4, b4, c4, s, o4);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    done = n4 * 4;
  }
  if (done < n) {
    hipLaunchKernelGGL(ew_scalar<OP>, dim3(grid_for(n - done)), dim3(256), 0, st, done, n, a, b, c, s, o);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace

namespace bch {

hipError_t launch_elementwise(hipStream_t s, int op, long long n, const float* a, const float* b, const float* c,
                              float scalar, float* out) {
  if (n <= 0) return hipSuccess;
  switch (op) {
    case kEwAdd: return launch_op<kEwAdd>(s, n, a, b, c, scalar, out);
    case kEwSub: return launch_op<kEwSub>(s, n, a, b, c, scalar, out);
    case kEwMul: return launch_op<kEwMul>(s, n, a, b, c, scalar, out);
    case kEwNeg: return launch_op<kEwNeg>(s, n, a, b, c, scalar, out);
    case kEwFma: return launch_op<kEwFma>(s, n, a, b, c, scalar, out);
    case kEwScale: return launch_op<kEwScale>(s, n, a, b, c, scalar, out);
    case kEwRelu: return launch_op<kEwRelu>(s, n, a, b, c, scalar, out);
    case kEwGelu: return launch_op<kEwGelu>(s, n, a, b, c, scalar, out);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bch
