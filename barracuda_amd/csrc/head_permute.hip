// head_permute.hip -- TensorSession::head_split / head_concat for gfx950.
//
// Replaces shaders/tensor/head_split_f64.wgsl ([B, S, H*D] -> [B, H, S, D],
// one thread per output element: out[b][h][s][d] = in[b][s][h*D + d]) and
// head_concat_f64.wgsl (the inverse map), which the reference session
// dispatches for SessionOp::HeadSplit / HeadConcat (crates/barracuda/src/
// session/dispatch.rs:332-389; recorded by session/mod.rs:423-480).
//
// Both are one batched transpose of a P x Q grid of D-vectors:
//   out[b][p][q][:] = in[b][q][p][:]
// with (P, Q) = (H, S) for head_split and (S, H) for head_concat.  A copy:
// HBM-bound at 8 bytes per element (one read, one write), no arithmetic.
// Workgroup row y of the grid owns one (b, p) and writes its Q*D outputs,
// which are contiguous; lane reads come in runs of D contiguous floats (one
// source row per q).  Each thread moves 4 float4 (or 4 floats when D % 4 != 0
// or a buffer is misaligned), all loads issued before the stores; tensors
// that move >= 64 MB use non-temporal loads and stores, like the element-wise
// kernels.
#include "bch_internal.h"

namespace {

constexpr int kPerThread = 4;  // vectors per thread
constexpr int kTpb = 256;
constexpr long long kNtBytes = 64LL << 20;

template <typename V, bool NT>
__device__ __forceinline__ V ld(const V* p) {
  if constexpr (NT && sizeof(V) == 16) return bch::load_nt(reinterpret_cast<const float4*>(p));
  else if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename V, bool NT>
__device__ __forceinline__ void st(V v, V* p) {
  if constexpr (NT && sizeof(V) == 16) bch::store_nt(v, reinterpret_cast<float4*>(p));
  else if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// V: float4 (dv = D / 4 vectors a row) or float (dv = D).  row = Q * dv
// vectors of one (b, p), 32-bit offsets inside it (the host checks Q * dv <
// 2^31).  Grid: x over the row in chunks of kTpb * kPerThread, y over b * P +
// p (striding by gridDim.y past 65535).
template <typename V, bool NT>
__global__ __launch_bounds__(kTpb) void head_permute_kernel(const V* __restrict__ in, V* __restrict__ out,
                                                            long long BP, int P, int Q, int dv) {
  const unsigned row = (unsigned)Q * (unsigned)dv;
  const unsigned j0 = blockIdx.x * (unsigned)(kTpb * kPerThread) + threadIdx.x;
  for (long long y = blockIdx.y; y < BP; y += gridDim.y) {
    const long long b = y / P, p = y - b * P;
    const V* src = in + (b * Q * P + p) * dv;  // + (q P) dv + c
    V* dst = out + y * (long long)row;          // + q dv + c
    V v[kPerThread];
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const unsigned j = j0 + u * kTpb;
      if (j < row) {
        const unsigned q = j / (unsigned)dv, c = j - q * (unsigned)dv;
        v[u] = ld<V, NT>(src + (long long)q * P * dv + c);
      }
    }
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const unsigned j = j0 + u * kTpb;
      if (j < row) st<V, NT>(v[u], dst + j);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename V>
hipError_t launch_v(hipStream_t s, long long BP, int P, int Q, int dv, const float* in, float* out, bool nt) {
  const long long row = (long long)Q * dv;
  const long long bx = (row + kTpb * kPerThread - 1) / (kTpb * kPerThread);
  const dim3 grid((unsigned)bx, (unsigned)(BP < 65535 ? BP : 65535));
  const V* i = reinterpret_cast<const V*>(in);
  V* o = reinterpret_cast<V*>(out);
  if (nt)
    hipLaunchKernelGGL((head_permute_kernel<V, true>), grid, dim3(kTpb), 0, s, i, o, BP, P, Q, dv);
  else
    hipLaunchKernelGGL((head_permute_kernel<V, false>), grid, dim3(kTpb), 0, s, i, o, BP, P, Q, dv);
  return hipGetLastError();
}

}  // namespace

namespace bch {

hipError_t launch_head_permute(hipStream_t s, bool concat, int B, int S, int H, int D, const float* in,
                               float* out) {
  if (B < 1 || S < 1 || H < 1 || D < 1) return hipSuccess;
  const int P = concat ? S : H, Q = concat ? H : S;
  const bool vec = D % 4 == 0 && aligned16(in) && aligned16(out);
  const int dv = vec ? D / 4 : D;
  if ((long long)Q * dv > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long bytes = 8LL * B * S * H * D;
  const bool nt = bytes >= kNtBytes;
  const long long BP = (long long)B * P;
  return vec ? launch_v<float4>(s, BP, P, Q, dv, in, out, nt) : launch_v<float>(s, BP, P, Q, dv, in, out, nt);
}

}  // namespace bch
