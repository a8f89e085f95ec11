// layer_norm.hip -- layer normalisation over the last axis for gfx950.
//
// Replaces TensorSession::layer_norm (crates/barracuda/src/session/mod.rs:
// 379-398, dispatched at session/dispatch.rs:221-240 with epsilon 1e-5) and
// the op it binds, LayerNorm (ops/layer_norm_wgsl.rs, shaders/norm/
// layer_norm_f64.wgsl: one thread per row, three sweeps).  Same contract per
// row of `cols` features, no affine parameters:
//   mean = sum(x) / cols
//   var  = sum((x - mean)^2) / cols          (two-pass, biased)
//   y    = (x - mean) / sqrt(var + eps)
//
// HBM-bound: one read and one write of the matrix (8 bytes per element).
//   * cols % 4 == 0, cols <= 4096, 16-byte aligned rows: one wavefront per
//     row; the row is loaded once with 128-bit coalesced loads and stays in
//     registers; the sum and the sum of squared deviations are wavefront
//     all-reductions (DPP row ops + v_readlane), so the two passes of the
//     reference cost no second read; the output is written once.
//   * 4096 < cols <= 65536, cols % 4 == 0, aligned: one workgroup per row,
//     8 / 16 / 32 float4 per thread in registers (1024 threads with 16 each
//     above 32768), block reductions; read once, write once.
//   * other widths (cols % 4 != 0, or unaligned) up to 32768: one workgroup
//     per row with up to 32 elements per thread in registers, scalar loads;
//     read once.
//   * anything else: one 256-thread workgroup per row, the same two passes
//     with block reductions over further reads of the row (from cache).
#include "bch_internal.h"

#include <math.h>

namespace {

using bch::OpSum;
using bch::wave_allreduce;

template <int NV>
__global__ __launch_bounds__(256) void layer_norm_wave(const float* in, float* out, long long rows, int cols,
                                                       float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int nvec = cols >> 2;
  const float4* src = reinterpret_cast<const float4*>(in + row * (long long)cols);
  float4* dst = reinterpret_cast<float4*>(out + row * (long long)cols);
  float4 v[NV];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * 64 + lane;
    v[i] = idx < nvec ? bch::load_nt(src + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  }
  const float mean = wave_allreduce(s, OpSum()) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i * 64 + lane < nvec) {
      const float dx = v[i].x - mean, dy = v[i].y - mean, dz = v[i].z - mean, dw = v[i].w - mean;
      q += fmaf(dx, dx, dy * dy) + fmaf(dz, dz, dw * dw);
    }
  }
  const float var = wave_allreduce(q, OpSum()) / (float)cols;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * 64 + lane;
    if (idx < nvec)
      bch::store_nt(make_float4((v[i].x - mean) * rstd, (v[i].y - mean) * rstd, (v[i].z - mean) * rstd,
                                (v[i].w - mean) * rstd),
                    dst + idx);
  }
}

// Sum over the 256 threads of a workgroup; every thread gets it.  Must be
// reached by all threads of the block.
template <int NW = 4>
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_allreduce(v, OpSum());
  const int w = threadIdx.x >> 6;
  __syncthreads();  // sh may still be read from the previous call
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  if (NW == 4) return (sh[0] + sh[1]) + (sh[2] + sh[3]);
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += sh[i];
  return r;
}

__global__ __launch_bounds__(256) void layer_norm_block(const float* in, float* out, long long cols, float eps) {
  __shared__ float sh[4];
  const long long row = blockIdx.x;
  const float* x = in + row * cols;
  float* y = out + row * cols;
  float s = 0.0f;
  for (long long j = threadIdx.x; j < cols; j += 256) s += x[j];
  const float mean = block_sum(s, sh) / (float)cols;
  float q = 0.0f;
  for (long long j = threadIdx.x; j < cols; j += 256) {
    const float d = x[j] - mean;
    q = fmaf(d, d, q);
  }
  const float var = block_sum(q, sh) / (float)cols;
  const float rstd = 1.0f / sqrtf(var + eps);
  for (long long j = threadIdx.x; j < cols; j += 256) y[j] = (x[j] - mean) * rstd;
}

// 4096 < cols <= 4 NT NV (cols % 4 == 0, 16-byte aligned): one NT-thread workgroup per row (256, or
// 1024 above 32768 columns), thread t holding float4 t, t + NT, ... (NV of them) in registers, so the row is read once and written
// once; the sums are block reductions (wavefront all-reductions, then LDS).
template <int NV, int NT>
__global__ __launch_bounds__(NT) void layer_norm_wg(const float* in, float* out, int cols, float eps) {
  __shared__ float sh[NT / 64];
  const long long row = blockIdx.x;
  const int nvec = cols >> 2;
  const float4* src = reinterpret_cast<const float4*>(in + row * (long long)cols);
  float4* dst = reinterpret_cast<float4*>(out + row * (long long)cols);
  float4 v[NV];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * NT + (int)threadIdx.x;
    v[i] = idx < nvec ? bch::load_nt(src + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  }
  const float mean = block_sum<NT / 64>(s, sh) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i * NT + (int)threadIdx.x < nvec) {
      const float dx = v[i].x - mean, dy = v[i].y - mean, dz = v[i].z - mean, dw = v[i].w - mean;
      q += fmaf(dx, dx, dy * dy) + fmaf(dz, dz, dw * dw);
    }
  }
  const float var = block_sum<NT / 64>(q, sh) / (float)cols;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * NT + (int)threadIdx.x;
    if (idx < nvec)
      bch::store_nt(make_float4((v[i].x - mean) * rstd, (v[i].y - mean) * rstd, (v[i].z - mean) * rstd,
                                (v[i].w - mean) * rstd),
                    dst + idx);
  }
}

// Rows of any width up to NT NS that the float4 kernels cannot take (cols % 4 != 0, or unaligned
// buffers): one NT-thread workgroup per row, thread t holding elements t, t + NT, ... (NS of them)
// in registers; scalar loads, read once, write once.
template <int NS, int NT>
__global__ __launch_bounds__(NT) void layer_norm_wgs(const float* in, float* out, int cols, float eps) {
  __shared__ float sh[NT / 64];
  const float* x = in + (long long)blockIdx.x * cols;
  float* y = out + (long long)blockIdx.x * cols;
  float v[NS];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int j = i * NT + (int)threadIdx.x;
    v[i] = j < cols ? __builtin_nontemporal_load(x + j) : 0.0f;
    s += v[i];
  }
  const float mean = block_sum<NT / 64>(s, sh) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (i * NT + (int)threadIdx.x < cols) {
      const float d = v[i] - mean;
      q = fmaf(d, d, q);
    }
  }
  const float var = block_sum<NT / 64>(q, sh) / (float)cols;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int j = i * NT + (int)threadIdx.x;
    if (j < cols) __builtin_nontemporal_store((v[i] - mean) * rstd, y + j);
  }
}

// Scalar register kernel for a row of cols: (NS, NT) coded as NS * 10000 + NT, 0 above 32768.
int pick_wgs(long long cols) {
  if (cols <= 1024) return 4 * 10000 + 256;
  if (cols <= 4096) return 16 * 10000 + 256;
  if (cols <= 16384) return 16 * 10000 + 1024;
  if (cols <= 32768) return 32 * 10000 + 1024;
  return 0;
}

int pick_wg_nv(long long cols) {
  if (cols % 4 != 0 || cols <= 4096) return 0;
  if (cols <= 8192) return 8;
  if (cols <= 16384) return 16;
  if (cols <= 32768) return 32;
  if (cols <= 65536) return 64;  // 1024 threads, 16 float4 each
  return 0;
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
  return cols % 4 == 0 && pick_nv(cols) > 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(out) & 15) == 0;
}

// Which kernel a call runs: the wavefront-per-row register kernel (sel = NV),
// the workgroup-per-row float4 register kernel (sel = NV, 64 meaning 16 on
// 1024 threads), the scalar register kernel (sel = NS * 10000 + NT), or the
// block kernel.  The float4 kernels need 16-byte aligned buffers; the launch
// and the reported name both come from this one choice.
enum class LnKind { kWave, kWg, kWgs, kBlock };
struct LnPlan {
  LnKind kind;
  int sel;
};

LnPlan ln_plan(long long cols, const float* in, const float* out) {
  const bool al = (reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (wave_path(cols, in, out)) return {LnKind::kWave, pick_nv(cols)};
  if (pick_wg_nv(cols) > 0 && al) return {LnKind::kWg, pick_wg_nv(cols)};
  if (pick_wgs(cols) > 0) return {LnKind::kWgs, pick_wgs(cols)};
  return {LnKind::kBlock, 0};
}

// One launch over n rows (n <= kLnRowsPerLaunch).
hipError_t launch_rows(hipStream_t s, const LnPlan& p, long long n, long long cols, float eps, const float* in,
                       float* out) {
  const int c = (int)cols;
  switch (p.kind) {
    case LnKind::kWave: {
      const dim3 grid((unsigned)((n + 3) / 4)), block(256);
      switch (p.sel) {
        case 1: hipLaunchKernelGGL(layer_norm_wave<1>, grid, block, 0, s, in, out, n, c, eps); break;
        case 2: hipLaunchKernelGGL(layer_norm_wave<2>, grid, block, 0, s, in, out, n, c, eps); break;
        case 4: hipLaunchKernelGGL(layer_norm_wave<4>, grid, block, 0, s, in, out, n, c, eps); break;
        case 8: hipLaunchKernelGGL(layer_norm_wave<8>, grid, block, 0, s, in, out, n, c, eps); break;
        default: hipLaunchKernelGGL(layer_norm_wave<16>, grid, block, 0, s, in, out, n, c, eps); break;
      }
      break;
    }
    case LnKind::kWg: {
      const dim3 grid((unsigned)n), block(256);
      switch (p.sel) {
        case 8: hipLaunchKernelGGL((layer_norm_wg<8, 256>), grid, block, 0, s, in, out, c, eps); break;
        case 16: hipLaunchKernelGGL((layer_norm_wg<16, 256>), grid, block, 0, s, in, out, c, eps); break;
        case 32: hipLaunchKernelGGL((layer_norm_wg<32, 256>), grid, block, 0, s, in, out, c, eps); break;
        default: hipLaunchKernelGGL((layer_norm_wg<16, 1024>), grid, dim3(1024), 0, s, in, out, c, eps); break;
      }
      break;
    }
    case LnKind::kWgs: {
      const dim3 grid((unsigned)n);
      switch (p.sel) {
        case 40256: hipLaunchKernelGGL((layer_norm_wgs<4, 256>), grid, dim3(256), 0, s, in, out, c, eps); break;
        case 160256: hipLaunchKernelGGL((layer_norm_wgs<16, 256>), grid, dim3(256), 0, s, in, out, c, eps); break;
        case 161024: hipLaunchKernelGGL((layer_norm_wgs<16, 1024>), grid, dim3(1024), 0, s, in, out, c, eps); break;
        default: hipLaunchKernelGGL((layer_norm_wgs<32, 1024>), grid, dim3(1024), 0, s, in, out, c, eps); break;
      }
      break;
    }
    default:
      hipLaunchKernelGGL(layer_norm_block, dim3((unsigned)n), dim3(256), 0, s, in, out, cols, eps);
      break;
  }
  return hipGetLastError();
}

}  // namespace

namespace bch {

const char* layer_norm_kernel_name(long long rows, long long cols, const float* in, const float* out) {
  (void)rows;
  const LnPlan p = ln_plan(cols, in, out);
  switch (p.kind) {
    case LnKind::kWave:
      switch (p.sel) {
        case 1: return "layer_norm_wave<1>";
        case 2: return "layer_norm_wave<2>";
        case 4: return "layer_norm_wave<4>";
        case 8: return "layer_norm_wave<8>";
        default: return "layer_norm_wave<16>";
      }
    case LnKind::kWg:
      switch (p.sel) {
        case 8: return "layer_norm_wg<8>";
        case 16: return "layer_norm_wg<16>";
        case 32: return "layer_norm_wg<32>";
        default: return "layer_norm_wg<16, 1024>";
      }
    case LnKind::kWgs:
      switch (p.sel) {
        case 40256: return "layer_norm_wgs<4, 256>";
        case 160256: return "layer_norm_wgs<16, 256>";
        case 161024: return "layer_norm_wgs<16, 1024>";
        default: return "layer_norm_wgs<32, 1024>";
      }
    default:
      return "layer_norm_block";
  }
}

long long row_launches(long long rows) { return rows <= 0 ? 0 : (rows + kRowsPerLaunch - 1) / kRowsPerLaunch; }

hipError_t launch_layer_norm(hipStream_t s, long long rows, long long cols, float eps, const float* in, float* out) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const LnPlan p = ln_plan(cols, in, out);
  // rows in launches of at most kRowsPerLaunch, so that no grid reaches 2^32
  // threads (up to 1024 a row); a chunk starts a whole number of rows in, so
  // the buffers' 16-byte alignment is kept where the float4 kernels need it
  for (long long r0 = 0; r0 < rows; r0 += kRowsPerLaunch) {
    const long long n = rows - r0 < kRowsPerLaunch ? rows - r0 : kRowsPerLaunch;
    const hipError_t e = launch_rows(s, p, n, cols, eps, in + r0 * cols, out + r0 * cols);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace bch
