// bch_internal.h -- launchers shared between the C-ABI (bch_runtime.hip) and
// the kernel translation units.  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace bch {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 128-bit loads/stores with the non-temporal hint (streamed once; keep them
// from displacing reusable lines in L2 / the Infinity Cache).
__device__ __forceinline__ float4 load_nt(const float4* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(float4 r, float4* p) {
  const f32x4 v = {r.x, r.y, r.z, r.w};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
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

// Activation of the linear layer's epilogue and of the element-wise ops
// (the values of BCH_ACT_*).
constexpr int kActNone = 0, kActRelu = 1, kActGelu = 2;

// GELU, tanh form (shaders/activation/gelu_f64.wgsl: 0.5 x (1 + tanh(y)),
// y = 0.7978845608 (x + 0.044715 x^3)), evaluated as the identical
// x / (1 + e^z), z = -2y, which stays finite for every finite x (an
// exp-ratio tanh such as the f64 shader's tanh_f64, math_f64.wgsl:718-722,
// overflows to inf/inf).  z > 88 (x below about -9.6): the quotient is below
// 1e-37 in magnitude and the result is -0 (also for x = -inf, where the
// formula itself is inf * 0).  z is floored at -126, where e^z already
// underflows to 0, so y = +inf (x^3 overflowing for |x| > 1.8e19) gives x.
// e^z is 2^(z log2 e) on v_exp_f32 with the product's rounding error carried
// by one fma (within a few ulp of a correctly rounded expf).  NaN propagates.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float y = 0.7978845608f * fmaf(0.044715f * x, x * x, x);
  float z = -2.0f * y;
  if (z > 88.0f) return -0.0f;
  z = z < -126.0f ? -126.0f : z;
  const float p = z * 1.44269502162933349609375f;
  float e = fmaf(z, 1.44269502162933349609375f, -p);
  e = fmaf(z, 1.925963033500011829e-8f, e);
  const float r = __builtin_amdgcn_exp2f(p);
  const float ez = fmaf(r, e * 0.693147180559945309f, r);
  return x / (1.0f + ez);
}

__device__ __forceinline__ float activate(float v, int act) {
  if (act == kActRelu) return fmaxf(v, 0.0f);
  if (act == kActGelu) return gelu_tanh(v);
  return v;
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

// Row softmax over a contiguous [rows, cols] f32 matrix (in may equal out).
// ws/ws_bytes: device scratch of at least softmax_workspace_bytes(rows, cols)
// bytes (zero when few long rows are not split across workgroups).  guard:
// a row whose sum is not > 0 (NaN, +inf or only -inf in it) keeps its
// exp(x - max) un-normalised, as Tensor::softmax_dim's host loop does;
// without it the row is divided like any other (all NaN).
hipError_t launch_softmax_rows(hipStream_t s, long long rows, long long cols,
                               const float* in, float* out, void* ws,
                               size_t ws_bytes, bool guard = false);
size_t softmax_workspace_bytes(long long rows, long long cols);
// Softmax along the middle axis of [outer, axis, inner]; the scratch rule of
// launch_softmax_rows applies when inner == 1, and guard as there.
hipError_t launch_softmax_axis(hipStream_t s, long long outer, long long axis,
                               long long inner, const float* in, float* out,
                               void* ws, size_t ws_bytes, bool guard = false);
size_t softmax_axis_workspace_bytes(long long outer, long long axis,
                                    long long inner);
// The row softmax (guard off) of x * scale with a causal mask, the scaled
// scores of an attention pass: row r of [rows][cols] holds the keys of query
// r0 + r % m, and with causal its columns past that query are -inf.  One
// pass, the wavefront-per-row kernel; only where softmax_rows_scaled_supported
// (cols % 4 == 0, cols <= 4096, 16-byte aligned buffers), else an error.
bool softmax_rows_scaled_supported(long long cols, const float* in, const float* out);
hipError_t launch_softmax_rows_scaled(hipStream_t s, long long rows, long long cols, const float* in, float* out,
                                      float scale, int causal, int m, int r0);
// The kernel a launch_softmax_rows with these buffers runs (the split plan's
// write kernel when few long rows are split).
const char* softmax_kernel_name(long long rows, long long cols, const float* in, const float* out);
// Row softmax over a contiguous [rows, cols] f64 matrix (in may equal out);
// no scratch.  aligned16: both matrices 16-byte aligned.
hipError_t launch_softmax_rows_f64(hipStream_t s, long long rows, long long cols,
                                   const double* in, double* out);
const char* softmax_f64_kernel_name(long long rows, long long cols,
                                    bool aligned16);

// C[b] = A[b] . B[b] (row-major), b < batch.  ws/ws_bytes: device scratch
// of at least sgemm_workspace_bytes(batch, m, n, k) bytes.
hipError_t launch_sgemm(hipStream_t s, int batch, int m, int n, int k,
                        const float* A, int lda, long long sA,
                        const float* B, int ldb, long long sB,
                        float* C, int ldc, long long sC, void* ws,
                        size_t ws_bytes);
size_t sgemm_workspace_bytes(int batch, int m, int n, int k);
// The part of it a launch cannot do without (the skinny paths' and split-K's
// partials); with less than sgemm_workspace_bytes the hybrid plan is skipped.
size_t sgemm_required_workspace_bytes(int batch, int m, int n, int k);
// Scratch of launch_sgemm_ex (the skinny paths' partials, split-K partials, or the hybrid plan's).
size_t sgemm_ex_workspace_bytes(bool transb, int batch, int m, int n, int k, int lda, int ldb);
const char* sgemm_kernel_name(int m, int n, int k);
// With B given as [n][k] when transb (C = A B^T), and the linear layer's
// epilogue C = act(acc + bias[col]): bias nullable, act kActNone / kActRelu /
// kActGelu.
hipError_t launch_sgemm_ex(hipStream_t s, bool transb, int batch, int m,
                           int n, int k, const float* A, int lda,
                           long long sA, const float* B, int ldb,
                           long long sB, const float* bias, int act,
                           float* C, int ldc, long long sC, void* ws,
                           size_t ws_bytes);

// Skinny (m <= 64; above 32 with K % 4 == 0 and 16-byte aligned A) GEMM: streams B once; split-k partials go to ws; the
// reduce applies the epilogue (bias nullable, act as above).
hipError_t launch_sgemm_skinny(hipStream_t s, int m, int n, int k,
                               const float* A, int lda, const float* B,
                               int ldb, float* C, int ldc, void* ws,
                               size_t ws_bytes, const float* bias, int act);
size_t sgemm_skinny_workspace_bytes(int m, int n, int k);
// Skinny (m <= 32) GEMM with W given as [n][k] (C = A W^T), same epilogue.
hipError_t launch_sgemm_skinny_nt(hipStream_t s, int m, int n, int k,
                                  const float* A, int lda, const float* W,
                                  int ldw, float* C, int ldc, void* ws,
                                  size_t ws_bytes, const float* bias, int act);
size_t sgemm_skinny_nt_workspace_bytes(int m, int n, int k);
bool sgemm_skinny_nt_applies(int m, int n, int k, const float* A, int lda,
                             const float* W, int ldw);
const char* sgemm_skinny_kernel_name(int m);
bool sgemm_skinny_applies(int m, int n, int k, const float* A, int lda,
                          const float* B, int ldb);

// f64 GEMM on the FP64 matrix cores: C[b] = alpha op(A[b]) op(B[b]) (+ beta
// C[b] when beta != 0); transa: A stored [k][m]; transb: B stored [n][k].
// ws/ws_bytes: device scratch of at least dgemm_workspace_bytes(batch, m, n,
// k) bytes (the split-k partials; zero when k is not split).
hipError_t launch_dgemm(hipStream_t s, bool transa, bool transb, int batch,
                        int m, int n, int k, double alpha, const double* A,
                        int lda, long long sA, const double* B, int ldb,
                        long long sB, double beta, double* C, int ldc,
                        long long sC, void* ws, size_t ws_bytes);
size_t dgemm_workspace_bytes(int batch, int m, int n, int k);
int dgemm_split_count(int batch, int m, int n, int k);

// Seeded fills (rng.rs LCG / lattice Box-Muller); state is the value before.
hipError_t launch_fill_uniform(hipStream_t s, float* out, uint64_t n, uint64_t state, double lo,
                               double hi);
hipError_t launch_fill_normal(hipStream_t s, float* out, uint64_t n, uint64_t state, double mu,
                              double sigma);
uint64_t lcg_advance(uint64_t state, uint64_t inc, uint64_t n);

// Launch controls of the calling context, set by the C ABI on the calling
// thread before a call's launches (a context's calls run on the thread that
// makes them, one at a time).  fault: a device-visible word in pinned host
// memory that the [out, in] skinny GEMM's in-kernel split-k combine sets when
// an owner gives up waiting for a contributor (its outputs are then NaN);
// the context reports BCH_E_DEVICE_LOST at its next synchronisation and
// every later call.  spin: that wait's poll limit (0 gives up at once: a
// host-side way to force the path in tests, every kernel still exiting).
struct LaunchCtl {
  unsigned* fault = nullptr;
  unsigned spin = 1u << 22;
};
LaunchCtl& launch_ctl();

// Compute units of the current device, cached per device; kDefaultCUs
// (MI355X) when no device is visible, so launch plans and kernel names can
// be computed without a GPU.
constexpr int kDefaultCUs = 256;
int device_cu_count();

// Raise `func`'s dynamic LDS limit to `bytes` on the current device, once per
// (function, device); thread-safe.  Kernels asking for more than 64 KB of
// dynamic LDS need it before their first launch on each device.
hipError_t ensure_dynamic_lds(const void* func, int bytes);

// Element-wise ops of the session (op: BCH_EW_*), HBM-streaming.
hipError_t launch_elementwise(hipStream_t s, int op, long long n, const float* a, const float* b,
                              const float* c, float scalar, float* out);
// Layer norm over the last axis of [rows, cols]: (x - mean) / sqrt(var + eps).
hipError_t launch_layer_norm(hipStream_t s, long long rows, long long cols, float eps, const float* in,
                             float* out);
// The kernel a launch_layer_norm with these buffers runs.
const char* layer_norm_kernel_name(long long rows, long long cols, const float* in, const float* out);

// Row kernels (softmax, layer norm) launch at most kRowsPerLaunch rows at a
// time: with up to 1024 threads a row, a grid then stays below 2^32 threads
// and 2^31 workgroups whatever the row count.  row_launches(rows) is the
// number of launches a call over `rows` rows makes.
constexpr long long kRowsPerLaunch = 1LL << 21;
long long row_launches(long long rows);

// head_split (concat false): [B, S, H*D] -> [B, H, S, D]; head_concat
// (concat true): the inverse.  in and out must not overlap.
hipError_t launch_head_permute(hipStream_t s, bool concat, int B, int S, int H, int D, const float* in,
                               float* out);

// Device-to-device copy (16-byte path when aligned).
hipError_t launch_copy(hipStream_t s, void* dst, const void* src, size_t bytes);

// Fused attention forward over [B,H,S,D].
hipError_t launch_sdpa(hipStream_t s, int B, int H, int Sq, int Skv, int D,
                       float scale, int causal, const float* q,
                       const float* k, const float* v, float* o);
// Strided form: per tensor (batch, head, row) strides in elements, the head
// dimension contiguous; key/value head of query head h is h / (H / Hkv).
struct SdpaLayout {
  long long batch, head, row;
};
struct SdpaStrides {
  SdpaLayout q, k, v, o;
};
// The fused kernel serves D <= kSdpaFusedMaxD.
constexpr int kSdpaFusedMaxD = 256;
hipError_t launch_sdpa_strided(hipStream_t s, int B, int H, int Hkv, int Sq,
                               int Skv, int D, float scale, int causal,
                               const float* q, const float* k,
                               const float* v, float* o,
                               const SdpaStrides& st);
// D > kSdpaFusedMaxD: scores materialised one query chunk at a time (GEMM,
// scaled and masked row softmax, GEMM) in ws, which must hold
// sdpa_wide_workspace_bytes(...) bytes (q_row, k_row: the row strides of q
// and k; 0 when a row stride exceeds 2^31 - 1, which the launch rejects).
size_t sdpa_wide_workspace_bytes(int Hkv, int Sq, int Skv, int D, int causal,
                                 long long q_row, long long k_row);
hipError_t launch_sdpa_wide(hipStream_t s, int B, int H, int Hkv, int Sq,
                            int Skv, int D, float scale, int causal,
                            const float* q, const float* k, const float* v,
                            float* o, const SdpaStrides& st, void* ws,
                            size_t ws_bytes);

}  // namespace bch
