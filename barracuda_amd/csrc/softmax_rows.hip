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
//   * a few long rows (the global softmax of Tensor::softmax and the session
//     is one row of every element): each row is cut into chunks, one
//     workgroup per chunk.  Pass 1 writes each chunk's online (max, sum)
//     to scratch; pass 2 merges the row's chunk states in every workgroup
//     and writes its chunk.  Read, read, write: 12 bytes per element, with
//     the whole chip busy instead of one CU per row.
//   * 4096 < cols <= 65536, cols % 4 == 0, rows left whole: one workgroup
//     per row, 8 / 16 / 32 float4 per thread in registers (1024 threads with
//     16 each above 32768); read once.
//   * other widths (cols % 4 != 0, or unaligned) up to 32768, rows left
//     whole: one workgroup per row with up to 32 elements per thread in
//     registers, scalar loads; read once.
//   * anything else: one workgroup per row, an online (max, sum) pass and a
//     second read that writes; scalar loads, any cols.
//   * axis != last: each [axis][inner] slice is a column softmax.  With
//     inner % 4 == 0 and 16-byte aligned pointers, lanes take float4
//     columns: 8 lanes a row (a whole 128-byte line) in 512-thread
//     workgroups, or 4 / 2 / 1 lanes a row in 256-thread ones for narrow
//     inner, 64 rows a pass.  Where the axis fits in 32 float4 registers a
//     lane and the strips fill the CUs, the workgroup keeps its whole strip
//     in registers: read once, max and sum by xor shuffles and LDS, write
//     once.  Otherwise the axis is cut into chunks: a stats kernel from
//     registers, then a streaming kernel that merges the chunk states and
//     writes; with inner >= 1024 the three passes (stats, merge, write)
//     read whole 4 KB row segments instead.  Any other inner: scalar lanes
//     over 64-column strips, online states merged in LDS.  Block numbers are
//     renumbered so that each XCD reads a contiguous run of strips.
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

using bch::OpMax;
using bch::OpSum;
using bch::wave_allreduce;

// The factor that normalises a row (a column) of sum s: 1 / s, or 1 where `guard` is set and s
// is not > 0 (a NaN sum: the row holds NaN or +inf; or nothing but -inf).  With guard the slice
// then keeps its exp(x - max) un-normalised, as the host loop of Tensor::softmax_dim does
// (ops/tensor_axis_ops.rs:108-114, `if sum > 0.0`); without it the division makes it NaN, as the
// global softmax's shader does (softmax_simple_f64.wgsl:45-50).  Finite rows are unaffected.
__device__ __forceinline__ float norm_inv(float s, int guard) { return guard && !(s > 0.0f) ? 1.0f : 1.0f / s; }
__device__ __forceinline__ float4 norm_inv4(float4 s, int guard) {
  return make_float4(norm_inv(s.x, guard), norm_inv(s.y, guard), norm_inv(s.z, guard), norm_inv(s.w, guard));
}

// One wavefront per row, NV float4 per lane (cols <= 256 * NV, cols % 4 == 0).
// PRE (the attention scores of the wide path): each loaded x first becomes
// x * scale, or -inf where causal and its column is past key pr0 + (prow0 +
// row) % pm -- the same f32 values a separate scale-and-mask pass writes.
template <int NV, bool PRE = false>
__device__ __forceinline__ void softmax_rows_wave_body(
    const float* in, float* out, long long rows,
    int cols, int guard, float scale = 1.0f, int causal = 0, int pm = 1, long long prow0 = 0, int pr0 = 0) {
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
  if constexpr (PRE) {
    const int lim = causal ? pr0 + (int)((prow0 + row) % pm) : 0x7fffffff;  // last key kept
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c0 = 4 * (i * 64 + lane);
      v[i].x = c0 > lim ? ninf : v[i].x * scale;
      v[i].y = c0 + 1 > lim ? ninf : v[i].y * scale;
      v[i].z = c0 + 2 > lim ? ninf : v[i].z * scale;
      v[i].w = c0 + 3 > lim ? ninf : v[i].w * scale;
    }
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
  const float inv = norm_inv(s, guard);
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
    const float* in, float* out, long long rows,
    int cols, int guard) {
  softmax_rows_wave_body<NV>(in, out, rows, cols, guard);
}

template <int NV>
__global__ __launch_bounds__(256) void softmax_rows_wave_scaled(const float* in, float* out, long long rows, int cols,
                                                                float scale, int causal, int pm, long long prow0,
                                                                int pr0) {
  softmax_rows_wave_body<NV, true>(in, out, rows, cols, 0, scale, causal, pm, prow0, pr0);
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

// Merge the (max, sum) states of the 256 threads of a workgroup; every
// thread gets the result.  Must be reached by all threads of the block.
__device__ __forceinline__ void block_merge(float& m, float& s) {
  __shared__ float sm[4], ss[4];
  // wave-level merge: all-reduce the max, rescale, all-reduce the sum
  const float wm = wave_allreduce(m, OpMax());
  const float ws = wave_allreduce(m == -INFINITY ? 0.0f : s * exp_f32(m - wm), OpSum());
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = wm;
    ss[w] = ws;
  }
  __syncthreads();
  float M = sm[0], S = ss[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) merge_state(M, S, sm[i], ss[i]);
  m = M;
  s = S;
}

// One workgroup (256 threads) per row, any cols.
__global__ __launch_bounds__(256) void softmax_rows_block(
    const float* in, float* out, long long rows,
    long long cols, int guard) {
  const long long row = blockIdx.x;
  const float* x = in + row * cols;
  float* y = out + row * cols;
  float m = -INFINITY, s = 0.0f;
  for (long long j = threadIdx.x; j < cols; j += 256) online_push(m, s, x[j]);
  block_merge(m, s);
  const float inv = norm_inv(s, guard);
  for (long long j = threadIdx.x; j < cols; j += 256) y[j] = exp_f32(x[j] - m) * inv;
}

// Rows of 4096 < cols <= 4 NT NV (cols % 4 == 0, 16-byte aligned) that the split plan leaves
// whole: one NT-thread workgroup per row (256, or 1024 above 32768 columns), thread t holding
// float4 t, t + NT, ... (NV of them), so
// the row is read once and written once, as in the wavefront-per-row kernel; max and sum are
// wavefront all-reductions, then the wavefronts' values in LDS.
template <int NW, class Op>
__device__ __forceinline__ float block_allreduce_nw(float v, Op op, float* red) {
  v = wave_allreduce(v, op);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (NW == 4) return op(op(red[0], red[1]), op(red[2], red[3]));
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = op(r, red[i]);
  return r;
}

template <int NV, int NT>
__global__ __launch_bounds__(NT) void softmax_rows_wg(const float* in, float* out, int cols, int guard) {
  __shared__ float redm[NT / 64], reds[NT / 64];
  const long long row = blockIdx.x;
  const int nvec = cols >> 2;
  const float4* src = reinterpret_cast<const float4*>(in + row * (long long)cols);
  float4* dst = reinterpret_cast<float4*>(out + row * (long long)cols);
  const float ninf = -INFINITY;
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * NT + (int)threadIdx.x;
    v[i] = idx < nvec ? bch::load_nt(src + idx) : make_float4(ninf, ninf, ninf, ninf);
  }
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < NV; ++i) mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
  mx = block_allreduce_nw<NT / 64>(mx, OpMax(), redm);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i * NT + (int)threadIdx.x < nvec) {
      v[i] = make_float4(exp_f32(v[i].x - mx), exp_f32(v[i].y - mx), exp_f32(v[i].z - mx), exp_f32(v[i].w - mx));
      s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
  }
  s = block_allreduce_nw<NT / 64>(s, OpSum(), reds);
  const float inv = norm_inv(s, guard);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = i * NT + (int)threadIdx.x;
    if (idx < nvec) bch::store_nt(make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv), dst + idx);
  }
}

// Rows of any width up to NT NS that the float4 kernels cannot take (cols % 4 != 0, or unaligned
// buffers), left whole by the split plan: one NT-thread workgroup per row, thread t holding elements
// t, t + NT, ... (NS of them) in registers; scalar loads, read once, write once.
template <int NS, int NT>
__global__ __launch_bounds__(NT) void softmax_rows_wgs(const float* in, float* out, int cols, int guard) {
  __shared__ float redm[NT / 64], reds[NT / 64];
  const float* x = in + (long long)blockIdx.x * cols;
  float* y = out + (long long)blockIdx.x * cols;
  float v[NS];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int j = i * NT + (int)threadIdx.x;
    v[i] = j < cols ? __builtin_nontemporal_load(x + j) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = block_allreduce_nw<NT / 64>(mx, OpMax(), redm);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (i * NT + (int)threadIdx.x < cols) {
      v[i] = exp_f32(v[i] - mx);
      s += v[i];
    }
  }
  s = block_allreduce_nw<NT / 64>(s, OpSum(), reds);
  const float inv = norm_inv(s, guard);
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int j = i * NT + (int)threadIdx.x;
    if (j < cols) __builtin_nontemporal_store(v[i] * inv, y + j);
  }
}

// Scalar register kernel for a row of cols: (NS, NT) coded as NS * 10000 + NT, 0 above 32768 (64
// elements per thread on 1024 threads spill).
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

// Online update with four elements at once: one rescale per float4.
__device__ __forceinline__ void online_push4(float& m, float& s, float4 v) {
  const float vm = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
  if (vm > m) {
    s *= exp_f32(m - vm);  // m == -inf: exp_f32 clamps to 0, s was 0
    m = vm;
  }
  if (m != -INFINITY)  // NaN elements make s NaN, as in online_push
    s += (exp_f32(v.x - m) + exp_f32(v.y - m)) + (exp_f32(v.z - m) + exp_f32(v.w - m));
}

// Split rows, pass 1: block (c, r) reduces chunk c of row r to (max, sum)
// and stores it at part[2 * (r * gridDim.x + c)].  VEC: float4 loads
// (cols % 4 == 0, 16-byte aligned input, chunk % 1024 == 0).
template <bool VEC>
__global__ __launch_bounds__(256) void softmax_split_stats(
    const float* __restrict__ in, long long cols, long long chunk,
    float* __restrict__ part) {
  const long long r = blockIdx.y;
  const long long j0 = (long long)blockIdx.x * chunk;
  const long long j1 = j0 + chunk < cols ? j0 + chunk : cols;
  const float* x = in + r * cols;
  float m = -INFINITY, s = 0.0f;
  if (VEC) {
    // four independent 16-byte loads in flight per thread before the math.
    // Ordinary (temporal) loads: what stays in the Infinity Cache serves part
    // of pass 2's re-read.  Measured on one 2^27-element row: 287 -> 272 us
    // per call; temporal loads in pass 2 as well 303 us; pass 2 walking each
    // chunk backwards 277 us.
    for (long long j = j0 + 4 * threadIdx.x; j < j1; j += 4096) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = j + 1024 * u < j1 ? *reinterpret_cast<const float4*>(x + j + 1024 * u)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (j + 1024 * u < j1) online_push4(m, s, v[u]);
    }
  } else {
    for (long long j = j0 + threadIdx.x; j < j1; j += 256) online_push(m, s, x[j]);
  }
  block_merge(m, s);
  if (threadIdx.x == 0) {
    const long long p = 2 * (r * gridDim.x + blockIdx.x);
    part[p] = m;
    part[p + 1] = s;
  }
}

// Split rows, pass 2: block (c, r) merges the gridDim.x chunk states of row
// r and writes chunk c.  VEC as in pass 1, plus a 16-byte aligned output.
template <bool VEC>
__global__ __launch_bounds__(256) void softmax_split_write(
    const float* in, float* out, long long cols,
    long long chunk, const float* __restrict__ part, int guard) {
  const long long r = blockIdx.y;
  const float* pr = part + 2 * r * gridDim.x;
  float m = -INFINITY, s = 0.0f;
  for (unsigned c = threadIdx.x; c < gridDim.x; c += 256) merge_state(m, s, pr[2 * c], pr[2 * c + 1]);
  block_merge(m, s);
  const float inv = norm_inv(s, guard);
  const long long j0 = (long long)blockIdx.x * chunk;
  const long long j1 = j0 + chunk < cols ? j0 + chunk : cols;
  const float* x = in + r * cols;
  float* y = out + r * cols;
  if (VEC) {
    for (long long j = j0 + 4 * threadIdx.x; j < j1; j += 4096) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = j + 1024 * u < j1 ? bch::load_nt(reinterpret_cast<const float4*>(x + j + 1024 * u))
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (j + 1024 * u < j1) {
          const float4 o = make_float4(exp_f32(v[u].x - m) * inv, exp_f32(v[u].y - m) * inv,
                                       exp_f32(v[u].z - m) * inv, exp_f32(v[u].w - m) * inv);
          bch::store_nt(o, reinterpret_cast<float4*>(y + j + 1024 * u));
        }
      }
    }
  } else {
    for (long long j = j0 + threadIdx.x; j < j1; j += 256) y[j] = exp_f32(x[j] - m) * inv;
  }
}

// Softmax along the middle axis of [outer, axis, inner]: X[o] = in + o axis inner is an
// [axis][inner] matrix (inner contiguous) and every column is one softmax.  Workgroup
// (o, chunk, strip), strip fastest, covers columns strip cw .. strip cw + cw - 1 (cw = 64, or
// inner when it is smaller) of the chunk's rows; thread (g, c), g < 256 / cw, takes rows
// g, g + 256 / cw, ... of column c, so each wavefront reads contiguous memory: 64 columns of one
// row, or 64 / inner whole rows.  The threads' online (max, sum) states meet in LDS and are
// merged in g order.  ONE: the chunk is the whole axis, and the workgroup goes on to write the
// column's outputs (read, read, write); otherwise it stores the chunk's state per column, and
// softmax_cols_write merges a column's chunk states in chunk order before writing its chunk.
struct ColWg {
  long long o;
  int chunk, strip;
};

// Workgroups are dispatched to the 8 XCDs round robin (block b to XCD b % 8); renumbering the
// first gridDim.x & ~7 blocks as (b % 8) * (that / 8) + b / 8 hands each XCD a contiguous run of
// strips, so the strips that share 128-byte lines of a row are read through the same L2.
__device__ __forceinline__ long long xcd_block() {
  const long long b = blockIdx.x, full = (long long)gridDim.x & ~7LL;
  return b < full ? (b & 7) * (full >> 3) + (b >> 3) : b;
}

__device__ __forceinline__ ColWg col_wg(int strips, int nchunks) {
  long long wg = xcd_block();
  ColWg r;
  r.strip = (int)(wg % strips);
  wg /= strips;
  r.chunk = (int)(wg % nchunks);
  r.o = wg / nchunks;
  return r;
}

template <bool ONE>
__global__ __launch_bounds__(256) void softmax_cols(const float* in, float* out, long long axis,
                                                    long long inner, int cw, int strips, int nchunks,
                                                    long long rpc, float* __restrict__ part, int guard) {
  __shared__ float sm[256], ss[256];
  const ColWg w = col_wg(strips, nchunks);
  const int rgs = 256 / cw;
  const int g = threadIdx.x / cw, c = threadIdx.x - g * cw;
  const long long col = (long long)w.strip * cw + c;
  const bool on = g < rgs && col < inner;
  const long long r0 = (long long)w.chunk * rpc, r1 = r0 + rpc < axis ? r0 + rpc : axis;
  const float* x = in + w.o * axis * inner + col;
  float m = -INFINITY, s = 0.0f;
  if (on) {
    long long r = r0 + g;
    for (; r + 3 * rgs < r1; r += 4 * rgs) {  // four independent loads before the math
      const float v0 = x[r * inner], v1 = x[(r + rgs) * inner], v2 = x[(r + 2 * rgs) * inner],
                  v3 = x[(r + 3 * rgs) * inner];
      online_push(m, s, v0);
      online_push(m, s, v1);
      online_push(m, s, v2);
      online_push(m, s, v3);
    }
    for (; r < r1; r += rgs) online_push(m, s, x[r * inner]);
  }
  sm[threadIdx.x] = m;
  ss[threadIdx.x] = s;
  __syncthreads();
  if (g == 0 && col < inner) {  // threads 0 .. cw - 1: merge the column's states in g order
    for (int gg = 1; gg < rgs; ++gg) merge_state(m, s, sm[gg * cw + c], ss[gg * cw + c]);
    if (ONE) {
      sm[c] = m;  // slot c is read by no other merging thread (they read slots >= cw)
      ss[c] = s;
    } else {
      const long long p = 2 * (((long long)w.o * nchunks + w.chunk) * inner + col);
      part[p] = m;
      part[p + 1] = s;
    }
  }
  if (!ONE) return;
  __syncthreads();
  if (!on) return;
  const float mx = sm[c], inv = norm_inv(ss[c], guard);
  float* y = out + w.o * axis * inner + col;
  for (long long r = r0 + g; r < r1; r += rgs) y[r * inner] = exp_f32(x[r * inner] - mx) * inv;
}

__global__ __launch_bounds__(256) void softmax_cols_write(const float* in, float* out, long long axis,
                                                          long long inner, int cw, int strips, int nchunks,
                                                          long long rpc, const float* __restrict__ part,
                                                          int guard) {
  const ColWg w = col_wg(strips, nchunks);
  const int rgs = 256 / cw;
  const int g = threadIdx.x / cw, c = threadIdx.x - g * cw;
  const long long col = (long long)w.strip * cw + c;
  if (g >= rgs || col >= inner) return;
  const float* pc = part + 2 * ((long long)w.o * nchunks * inner + col);
  float m = -INFINITY, s = 0.0f;
  for (int k = 0; k < nchunks; ++k) merge_state(m, s, pc[2LL * k * inner], pc[2LL * k * inner + 1]);
  const float inv = norm_inv(s, guard);
  const long long r0 = (long long)w.chunk * rpc, r1 = r0 + rpc < axis ? r0 + rpc : axis;
  const float* x = in + w.o * axis * inner + col;
  float* y = out + w.o * axis * inner + col;
  for (long long r = r0 + g; r < r1; r += rgs) y[r * inner] = exp_f32(x[r * inner] - m) * inv;
}

// Middle-axis softmax with a whole column strip in registers (inner % 4 == 0, 16-byte aligned,
// axis <= R * 256 / W): workgroup (o, strip) covers float4 columns strip W .. strip W + W - 1;
// lane (g, c), c < W, holds column strip W + c of rows g, g + 256 / W, ... as R float4, so x is
// read once and y written once.  A wavefront reads W * 16 bytes of each of 64 / W rows per load.
// The column's max, then its sum of exp(x - max), meet across the lanes of the column by xor
// shuffles within the wavefront (lanes l and l ^ kW share c), then across the four wavefronts in
// LDS in wavefront order.  Rows past the axis load as -inf and add exp(-inf) = 0.
template <int W, int NW>
__device__ __forceinline__ float4 col_reduce(float4 a, float4 (*red)[W], bool is_max) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = W; off < 64; off <<= 1) {
    const float4 b = make_float4(__shfl_xor(a.x, off), __shfl_xor(a.y, off), __shfl_xor(a.z, off),
                                 __shfl_xor(a.w, off));
    a = is_max ? make_float4(fmaxf(a.x, b.x), fmaxf(a.y, b.y), fmaxf(a.z, b.z), fmaxf(a.w, b.w))
               : make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
  if (lane < W) red[wv][lane] = a;
  __syncthreads();
  const int c = lane % W;
  float4 r = red[0][c];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    const float4 b = red[i][c];
    r = is_max ? make_float4(fmaxf(r.x, b.x), fmaxf(r.y, b.y), fmaxf(r.z, b.z), fmaxf(r.w, b.w))
               : make_float4(r.x + b.x, r.y + b.y, r.z + b.z, r.w + b.w);
  }
  return r;
}

template <int R, int W, int NT, bool STATS>
__global__ __launch_bounds__(NT) void softmax_cols_reg(const float* in, float* out, long long axis,
                                                       long long inner4, long long strips, long long nchunks,
                                                       float4* __restrict__ part, long long plane, int guard) {
  constexpr int kRpp = NT / W, kNW = NT / 64;
  __shared__ float4 redm[kNW][W], reds[kNW][W];
  const long long b = xcd_block();
  const long long t = b / strips, strip = b - t * strips;
  const long long o = t / nchunks, chunk = t - o * nchunks;
  const int c = threadIdx.x % W, g = threadIdx.x / W;
  const long long col4 = strip * W + c;
  const bool on = col4 < inner4;
  const long long r0 = chunk * (R * kRpp);
  const long long r1 = r0 + R * kRpp < axis ? r0 + R * kRpp : axis;
  const float4* x = reinterpret_cast<const float4*>(in) + o * axis * inner4 + col4;
  float4* y = reinterpret_cast<float4*>(out) + o * axis * inner4 + col4;
  const float ninf = -INFINITY;
  float4 v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const long long r = r0 + g + (long long)i * kRpp;
    v[i] = on && r < r1 ? bch::load_nt(x + r * inner4) : make_float4(ninf, ninf, ninf, ninf);
  }
  float4 mx = v[0];
#pragma unroll
  for (int i = 1; i < R; ++i)
    mx = make_float4(fmaxf(mx.x, v[i].x), fmaxf(mx.y, v[i].y), fmaxf(mx.z, v[i].z), fmaxf(mx.w, v[i].w));
  mx = col_reduce<W, kNW>(mx, redm, true);
  float4 sm = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    v[i] = make_float4(exp_f32(v[i].x - mx.x), exp_f32(v[i].y - mx.y), exp_f32(v[i].z - mx.z),
                       exp_f32(v[i].w - mx.w));
    sm = make_float4(sm.x + v[i].x, sm.y + v[i].y, sm.z + v[i].z, sm.w + v[i].w);
  }
  sm = col_reduce<W, kNW>(sm, reds, false);
  if (!on) return;
  if (STATS) {  // the chunk's (max, sum) per column; an all -inf chunk is the empty state (-inf, 0)
    if (g == 0) {
      const long long p = (o * nchunks + chunk) * inner4 + col4;
      part[p] = mx;
      part[plane + p] = make_float4(mx.x == ninf ? 0.0f : sm.x, mx.y == ninf ? 0.0f : sm.y,
                                    mx.z == ninf ? 0.0f : sm.z, mx.w == ninf ? 0.0f : sm.w);
    }
    return;
  }
  const float4 inv = norm_inv4(sm, guard);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const long long r = r0 + g + (long long)i * kRpp;
    if (r < r1)
      bch::store_nt(make_float4(v[i].x * inv.x, v[i].y * inv.y, v[i].z * inv.z, v[i].w * inv.w), y + r * inner4);
  }
}

// Second kernel of the chunked float4 path: row group g loads the column's states of chunks g,
// g + NT / W, ... (merged in that order), a shuffle-down tree merges them into lanes g == 0 of each
// wavefront, and every lane merges the wavefronts' states from LDS in wavefront order (the same
// order in every lane, so each lane of a column gets the same bits); then the workgroup writes its
// chunk of rows (rpc = R * NT / W rows) from a second read of x.
__device__ __forceinline__ void merge_state4(float4& m, float4& s, float4 m2, float4 s2) {
  merge_state(m.x, s.x, m2.x, s2.x);
  merge_state(m.y, s.y, m2.y, s2.y);
  merge_state(m.z, s.z, m2.z, s2.z);
  merge_state(m.w, s.w, m2.w, s2.w);
}

template <int W, int NT>
__global__ __launch_bounds__(NT) void softmax_cols_vwrite(const float* in, float* out, long long axis,
                                                          long long inner4, long long strips, long long nchunks,
                                                          long long rpc, const float4* __restrict__ part,
                                                          long long plane, int guard) {
  constexpr int kRpp = NT / W, kNW = NT / 64;
  __shared__ float4 stm[kNW][W], sts[kNW][W];
  const long long b = xcd_block();
  const long long t = b / strips, strip = b - t * strips;
  const long long o = t / nchunks, chunk = t - o * nchunks;
  const int c = threadIdx.x % W, g = threadIdx.x / W, lane = threadIdx.x & 63;
  const long long col4 = strip * W + c;
  const bool on = col4 < inner4;
  {
    float4 m = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY), sm = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (on) {
      const float4* pm = part + o * nchunks * inner4 + col4;
      for (long long k = g; k < nchunks; k += kRpp) merge_state4(m, sm, pm[k * inner4], pm[plane + k * inner4]);
    }
#pragma unroll
    for (int off = 32; off >= W; off >>= 1) {  // lanes < off take lane + off's state
      const float4 m2 = make_float4(__shfl_down(m.x, off), __shfl_down(m.y, off), __shfl_down(m.z, off),
                                    __shfl_down(m.w, off));
      const float4 s2 = make_float4(__shfl_down(sm.x, off), __shfl_down(sm.y, off), __shfl_down(sm.z, off),
                                    __shfl_down(sm.w, off));
      merge_state4(m, sm, m2, s2);
    }
    if (lane < W) {
      stm[threadIdx.x >> 6][lane] = m;
      sts[threadIdx.x >> 6][lane] = sm;
    }
  }
  __syncthreads();
  if (!on) return;
  float4 m = stm[0][c], sm = sts[0][c];
#pragma unroll
  for (int i = 1; i < kNW; ++i) merge_state4(m, sm, stm[i][c], sts[i][c]);
  const float4 inv = norm_inv4(sm, guard);
  const long long r0 = chunk * rpc, r1 = r0 + rpc < axis ? r0 + rpc : axis;
  const float4* x = reinterpret_cast<const float4*>(in) + o * axis * inner4 + col4;
  float4* y = reinterpret_cast<float4*>(out) + o * axis * inner4 + col4;
#pragma unroll 4
  for (long long r = r0 + g; r < r1; r += kRpp) {
    const float4 v = bch::load_nt(x + r * inner4);
    bch::store_nt(make_float4(exp_f32(v.x - m.x) * inv.x, exp_f32(v.y - m.y) * inv.y,
                              exp_f32(v.z - m.z) * inv.z, exp_f32(v.w - m.w) * inv.w),
                  y + r * inner4);
  }
}

// Float4 plan (inner % 4 == 0, 16-byte aligned): W lanes a row (float4 columns) in workgroups of
// NT threads, R float4 registers a lane, so R * NT / W rows a chunk.  Strips of 8 float4 (a whole
// 128-byte line of each row) in 512-thread workgroups where inner has 8 or more float4, so that no
// line is split between workgroups; 64 rows a pass either way.  One chunk when the axis fits in
// registers (R <= 32) and the strips fill the CUs: read once, write once.  Otherwise chunks of
// the largest R <= 16 that still gives 2 workgroups a CU (R >= 4; 16 rather than 32 keeps two
// 512-thread stats workgroups on a CU): a stats kernel and a write kernel.
struct VecPlan {
  int w = 0, nt = 256, r = 0;
  long long strips = 0, nchunks = 1, rpc = 0;
};

VecPlan vec_plan(long long outer, long long axis, long long inner) {
  VecPlan p;
  if (inner % 4 != 0) return p;
  const long long inner4 = inner / 4;
  const int w = inner4 >= 8 ? 8 : inner4 >= 3 ? 4 : (int)inner4;
  const int nt = w == 8 ? 512 : 256, rpp = nt / w;
  const long long strips = (inner4 + w - 1) / w;
  const long long cu = bch::device_cu_count();
  int r = 4;
  while (r < 32 && (long long)r * rpp < axis) r *= 2;
  if ((long long)r * rpp < axis || outer * strips < cu) {  // chunks: 2 workgroups a CU where possible
    r = 16;
    while (r > 4 && outer * strips * ((axis + (long long)r * rpp - 1) / ((long long)r * rpp)) < 2 * cu) r /= 2;
  }
  p.w = w;
  p.nt = nt;
  p.r = r;
  p.strips = strips;
  p.rpc = (long long)r * rpp;
  p.nchunks = (axis + p.rpc - 1) / p.rpc;
  if (outer * strips * p.nchunks > 0x7fffffffLL) p.w = 0;
  return p;
}

bool vec_aligned(const void* in, const void* out) {
  return (reinterpret_cast<uintptr_t>(in) % 16) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
}

template <int W, int NT, bool STATS>
void launch_cols_vec_r(hipStream_t s, const VecPlan& p, long long blocks, long long axis, long long inner4,
                       const float* in, float* out, float4* part, long long plane, int guard) {
  const dim3 grid((unsigned)blocks), block(NT);
  switch (p.r) {
    case 4: hipLaunchKernelGGL((softmax_cols_reg<4, W, NT, STATS>), grid, block, 0, s, in, out, axis, inner4, p.strips, p.nchunks, part, plane, guard); break;
    case 8: hipLaunchKernelGGL((softmax_cols_reg<8, W, NT, STATS>), grid, block, 0, s, in, out, axis, inner4, p.strips, p.nchunks, part, plane, guard); break;
    case 16: hipLaunchKernelGGL((softmax_cols_reg<16, W, NT, STATS>), grid, block, 0, s, in, out, axis, inner4, p.strips, p.nchunks, part, plane, guard); break;
    default: hipLaunchKernelGGL((softmax_cols_reg<32, W, NT, STATS>), grid, block, 0, s, in, out, axis, inner4, p.strips, p.nchunks, part, plane, guard); break;
  }
  if (STATS)
    hipLaunchKernelGGL((softmax_cols_vwrite<W, NT>), grid, block, 0, s, in, out, axis, inner4, p.strips, p.nchunks,
                       p.rpc, part, plane, guard);
}

template <int W, int NT>
void launch_cols_vec_w(hipStream_t s, const VecPlan& p, long long outer, long long axis, long long inner4,
                       const float* in, float* out, float4* part, int guard) {
  const long long blocks = outer * p.strips * p.nchunks;
  if (p.nchunks == 1)
    launch_cols_vec_r<W, NT, false>(s, p, blocks, axis, inner4, in, out, nullptr, 0, guard);
  else
    launch_cols_vec_r<W, NT, true>(s, p, blocks, axis, inner4, in, out, part, outer * p.nchunks * inner4, guard);
}

// ---- Wide rows, long axis: [outer, axis, inner] with inner >= 1024 (float4, aligned) and an
// axis too long for a column strip in registers.  The strips of the float4 plan (8 float4 of a row
// per workgroup, rows 8 KB apart at inner = 2048) streamed the write pass at 4.5 TB/s; here every
// pass reads whole rows: a workgroup of 256 threads covers 256 float4 columns (4 KB of a row) and
// walks a chunk of rows, so each wavefront touches 1 KB contiguous per row and the workgroup's rows
// follow each other in memory.
//   stats: per column, a running (max, sum) over the chunk's rows in register batches of kWideRb
//          rows (batch max, one rescale, batch sum), stored per chunk as (max, sum);
//   merge: per column, the chunks' states merged in a fixed order (kMergeSlots chunk slots a
//          column, each taking every kMergeSlots-th chunk, then a shuffle-down tree and the
//          wavefronts in order), stored as (max, 1 / sum);
//   write: per column, y = exp(x - max) / sum, streamed; write chunk c takes rows c, c + nchunks,
//          ..., so the workgroups in flight cover neighbouring rows (186 us against 194 us for
//          contiguous chunks at 1 x 65536 x 2048; the stats pass is faster on contiguous chunks).
// An all -inf chunk is the empty state (-inf, 0); NaN or +inf anywhere in a column makes its sum
// NaN, and the merge stores the normaliser norm_inv gives for it, as the float4 plan does.
constexpr int kWideCols = 256;  // float4 columns per workgroup (one per thread)
constexpr int kWideRb = 8;      // rows per register batch

struct WidePlan {
  bool on = false;
  long long ncb = 0, ch = 0, nchunks = 0;  // column blocks, rows per chunk, chunks
};

WidePlan wide_plan(long long outer, long long axis, long long inner) {
  WidePlan p;
  if (inner % 4 != 0 || inner / 4 < kWideCols) return p;
  const VecPlan vp = vec_plan(outer, axis, inner);
  if (vp.w == 0 || vp.nchunks == 1) return p;  // the strips fit in registers: read once, write once
  const long long inner4 = inner / 4;
  p.ncb = (inner4 + kWideCols - 1) / kWideCols;
  // about 4 workgroups a CU over the whole tensor, rows a multiple of the batch, 16..4096
  const long long target = 4LL * bch::device_cu_count();
  long long ch = (outer * p.ncb * axis + target - 1) / target;
  ch = (ch + kWideRb - 1) / kWideRb * kWideRb;
  ch = ch < 16 ? 16 : ch > 4096 ? 4096 : ch;
  p.ch = ch;
  p.nchunks = (axis + ch - 1) / ch;
  p.on = outer * p.nchunks * p.ncb <= 0x7fffffffLL && outer * inner4 <= 0x7fffffffLL;
  return p;
}

size_t wide_bytes(long long outer, long long inner, const WidePlan& p) {
  // per-chunk states (max, sum), then the merged (max, 1 / sum), all float4 per column
  return sizeof(float) * 2 * (size_t)outer * (size_t)inner * (size_t)(p.nchunks + 1);
}

__device__ __forceinline__ float4 max4(float4 a, float4 b) {
  return make_float4(fmaxf(a.x, b.x), fmaxf(a.y, b.y), fmaxf(a.z, b.z), fmaxf(a.w, b.w));
}

// running state (m, s) merged with a batch whose max is bm and whose values are v[0..n)
__device__ __forceinline__ void wide_batch(float& m, float& s, float bm, const float* v, int n) {
  const float mn = fmaxf(m, bm);
  if (mn == -INFINITY) return;  // all -inf so far: the empty state
  float acc = m == -INFINITY ? 0.0f : s * exp_f32(m - mn);
  for (int i = 0; i < n; ++i) acc += exp_f32(v[i] - mn);
  s = acc;
  m = mn;
}

__global__ __launch_bounds__(256) void softmax_cols_wide_stats(const float4* __restrict__ in, long long axis,
                                                               long long inner4, long long ncb, long long nchunks,
                                                               long long ch, float4* __restrict__ part,
                                                               long long plane) {
  const long long b = blockIdx.x;
  const long long cb = b % ncb, t = b / ncb, chunk = t % nchunks, o = t / nchunks;
  const long long col4 = cb * kWideCols + threadIdx.x;
  if (col4 >= inner4) return;
  const long long r0 = chunk * ch, r1 = r0 + ch < axis ? r0 + ch : axis;
  const float4* x = in + o * axis * inner4 + col4;
  const float ninf = -INFINITY;
  float4 m = make_float4(ninf, ninf, ninf, ninf), sm = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (long long r = r0; r < r1; r += kWideRb) {
    float4 v[kWideRb];
#pragma unroll
    for (int i = 0; i < kWideRb; ++i)
      v[i] = r + i < r1 ? bch::load_nt(x + (r + i) * inner4) : make_float4(ninf, ninf, ninf, ninf);
    float4 bm = v[0];
#pragma unroll
    for (int i = 1; i < kWideRb; ++i) bm = max4(bm, v[i]);
    float c[kWideRb];
#pragma unroll
    for (int i = 0; i < kWideRb; ++i) c[i] = v[i].x;
    wide_batch(m.x, sm.x, bm.x, c, kWideRb);
#pragma unroll
    for (int i = 0; i < kWideRb; ++i) c[i] = v[i].y;
    wide_batch(m.y, sm.y, bm.y, c, kWideRb);
#pragma unroll
    for (int i = 0; i < kWideRb; ++i) c[i] = v[i].z;
    wide_batch(m.z, sm.z, bm.z, c, kWideRb);
#pragma unroll
    for (int i = 0; i < kWideRb; ++i) c[i] = v[i].w;
    wide_batch(m.w, sm.w, bm.w, c, kWideRb);
  }
  const long long p = (o * nchunks + chunk) * inner4 + col4;
  part[p] = m;
  part[plane + p] = sm;
}

// A workgroup of 256 merges kMergeCols adjacent float4 columns q (of one outer index): thread t
// takes column t % kMergeCols and chunk slot j = t / kMergeCols, i.e. chunks j, j + kMergeSlots,
// ..., so a wavefront's loads are runs of kMergeCols * 16 bytes; a shuffle-down tree over the
// slots of a wavefront and then the four wavefronts, in order, finish each column.  Workgroups
// are renumbered XCD-major (xcd_block), so the workgroups whose columns share 128-byte lines read
// them through one L2.  fin[q] = max, fin[nq + q] = 1 / sum.
constexpr int kMergeCols = 1;
constexpr int kMergeSlots = 256 / kMergeCols;
__global__ __launch_bounds__(256) void softmax_cols_wide_merge(const float4* __restrict__ part, long long plane,
                                                               long long nchunks, long long inner4, long long nq,
                                                               float4* __restrict__ fin, int guard) {
  __shared__ float4 wm[4][kMergeCols], wsum[4][kMergeCols];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, c = threadIdx.x % kMergeCols;
  const long long per = (inner4 + kMergeCols - 1) / kMergeCols;  // column groups of one outer index
  const long long b = xcd_block();
  const long long o = b / per, col4 = (b - o * per) * kMergeCols + c;
  const float ninf = -INFINITY;
  float4 m = make_float4(ninf, ninf, ninf, ninf), sm = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (col4 < inner4) {
    const float4* pm = part + o * nchunks * inner4 + col4;
    for (long long k = threadIdx.x / kMergeCols; k < nchunks; k += kMergeSlots)
      merge_state4(m, sm, pm[k * inner4], pm[plane + k * inner4]);
  }
#pragma unroll
  for (int off = 32; off >= kMergeCols; off >>= 1) {  // lanes < off take lane + off's state
    const float4 m2 = make_float4(__shfl_down(m.x, off), __shfl_down(m.y, off), __shfl_down(m.z, off),
                                  __shfl_down(m.w, off));
    const float4 s2 = make_float4(__shfl_down(sm.x, off), __shfl_down(sm.y, off), __shfl_down(sm.z, off),
                                  __shfl_down(sm.w, off));
    merge_state4(m, sm, m2, s2);
  }
  if (lane < kMergeCols) {
    wm[w][lane] = m;
    wsum[w][lane] = sm;
  }
  __syncthreads();
  if (threadIdx.x < kMergeCols && col4 < inner4) {
    m = wm[0][c];
    sm = wsum[0][c];
#pragma unroll
    for (int i = 1; i < 4; ++i) merge_state4(m, sm, wm[i][c], wsum[i][c]);
    const long long q = o * inner4 + col4;
    fin[q] = m;
    fin[nq + q] = norm_inv4(sm, guard);
  }
}

__global__ __launch_bounds__(256) void softmax_cols_wide_write(const float4* __restrict__ in, float4* __restrict__ out,
                                                               long long axis, long long inner4, long long ncb,
                                                               long long nchunks, const float4* __restrict__ fin,
                                                               long long nq) {
  const long long b = blockIdx.x;
  const long long cb = b % ncb, t = b / ncb, chunk = t % nchunks, o = t / nchunks;
  const long long col4 = cb * kWideCols + threadIdx.x;
  if (col4 >= inner4) return;
  const long long q = o * inner4 + col4;
  const float4 m = fin[q], inv = fin[nq + q];
  const float4* x = in + o * axis * inner4 + col4;
  float4* y = out + o * axis * inner4 + col4;
#pragma unroll 8
  for (long long r = chunk; r < axis; r += nchunks) {
    const float4 v = bch::load_nt(x + r * inner4);
    bch::store_nt(make_float4(exp_f32(v.x - m.x) * inv.x, exp_f32(v.y - m.y) * inv.y,
                              exp_f32(v.z - m.z) * inv.z, exp_f32(v.w - m.w) * inv.w),
                  y + r * inner4);
  }
}

hipError_t launch_cols_wide(hipStream_t s, const WidePlan& p, long long outer, long long axis, long long inner,
                            const float* in, float* out, void* ws, int guard) {
  const long long inner4 = inner / 4, nq = outer * inner4;
  float4* part = static_cast<float4*>(ws);
  const long long plane = outer * p.nchunks * inner4;
  float4* fin = part + 2 * plane;
  const long long blocks = outer * p.nchunks * p.ncb;
  const float4* x = reinterpret_cast<const float4*>(in);
  hipLaunchKernelGGL(softmax_cols_wide_stats, dim3((unsigned)blocks), dim3(256), 0, s, x, axis, inner4, p.ncb,
                     p.nchunks, p.ch, part, plane);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long mblocks = outer * ((inner4 + kMergeCols - 1) / kMergeCols);
  hipLaunchKernelGGL(softmax_cols_wide_merge, dim3((unsigned)mblocks), dim3(256), 0, s, part, plane,
                     p.nchunks, inner4, nq, fin, guard);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(softmax_cols_wide_write, dim3((unsigned)blocks), dim3(256), 0, s, x,
                     reinterpret_cast<float4*>(out), axis, inner4, p.ncb, p.nchunks, fin, nq);
  return hipGetLastError();
}

// Chunking of the middle-axis softmax: enough workgroups for ~4 per CU, at least 256 rows a chunk.
struct ColPlan {
  int cw = 1, strips = 1, nchunks = 1;
  long long rpc = 1;
};

ColPlan col_plan(long long outer, long long axis, long long inner) {
  ColPlan p;
  p.cw = inner >= 64 ? 64 : (int)inner;
  p.strips = (int)((inner + p.cw - 1) / p.cw);
  const long long wgs = outer * p.strips;
  const long long target = 4LL * bch::device_cu_count();
  long long nc = 1;
  if (wgs < target) {
    nc = (target + wgs - 1) / wgs;
    const long long most = axis / 256 > 1 ? axis / 256 : 1;
    if (nc > most) nc = most;
  }
  p.rpc = (axis + nc - 1) / nc;
  p.nchunks = (int)((axis + p.rpc - 1) / p.rpc);
  return p;
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

// Split-row plan: rows that alone would leave most of the 256 CUs idle are
// cut into chunks of a multiple of 1024 elements (at least 16 Ki) so that
// about kSplitTarget workgroups run; at most kMaxSplits chunks per row.
// Measured on one 2^27-element row (both passes): 1024 / 2048 / 4096
// workgroups 287 / 293 / 302 us; 8 instead of 4 loads in flight per thread
// 290 us.
constexpr long long kSplitTarget = 1024;
constexpr long long kMinChunk = 16384;
constexpr long long kMaxSplits = 4096;

struct SplitPlan {
  long long splits = 1, chunk = 0;
};

SplitPlan split_plan(long long rows, long long cols) {
  SplitPlan p;
  if (pick_nv(cols) > 0 && (cols % 4) == 0) return p;  // wave path is one pass
  long long want = (kSplitTarget + rows - 1) / rows;
  long long most = (cols + kMinChunk - 1) / kMinChunk;
  long long sp = want < most ? want : most;
  if (sp > kMaxSplits) sp = kMaxSplits;
  if (sp < 2) return p;
  long long chunk = (cols + sp - 1) / sp;
  chunk = (chunk + 1023) / 1024 * 1024;
  p.splits = (cols + chunk - 1) / chunk;
  p.chunk = chunk;
  if (p.splits < 2) p.splits = 1;
  return p;
}

}  // namespace

namespace bch {

size_t softmax_workspace_bytes(long long rows, long long cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const SplitPlan p = split_plan(rows, cols);
  return p.splits > 1 ? (size_t)(2 * rows * p.splits) * sizeof(float) : 0;
}

size_t softmax_axis_workspace_bytes(long long outer, long long axis, long long inner) {
  if (inner == 1) return softmax_workspace_bytes(outer, axis);
  // the wide-row plan's, the float4 plan's chunks, or the scalar plan's when the pointers turn
  // out unaligned: the most any of them can take
  const WidePlan wp = wide_plan(outer, axis, inner);
  const ColPlan p = col_plan(outer, axis, inner);
  const VecPlan vp = vec_plan(outer, axis, inner);
  const long long nc = vp.w && vp.nchunks > p.nchunks ? vp.nchunks : p.nchunks;
  const size_t b = nc > 1 ? sizeof(float) * 2 * (size_t)outer * nc * (size_t)inner : 0;
  return wp.on && wide_bytes(outer, inner, wp) > b ? wide_bytes(outer, inner, wp) : b;
}

}  // namespace bch

namespace {

// Which kernel a row softmax that is not split runs: the wavefront-per-row
// register kernel (sel = NV), the workgroup-per-row float4 register kernel
// (sel = NV, 64 meaning 16 on 1024 threads), the scalar register kernel
// (sel = NS * 10000 + NT), or the block kernel.  The launch and the reported
// name both come from this one choice.
enum class SmKind { kWave, kWg, kWgs, kBlock };
struct SmPlan {
  SmKind kind;
  int sel;
};

SmPlan sm_plan(long long cols, const float* in, const float* out) {
  const bool al = (reinterpret_cast<uintptr_t>(in) % 16) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  if (wave_path(cols, in, out)) return {SmKind::kWave, pick_nv(cols)};
  if (pick_wg_nv(cols) > 0 && al) return {SmKind::kWg, pick_wg_nv(cols)};
  if (pick_wgs(cols) > 0) return {SmKind::kWgs, pick_wgs(cols)};
  return {SmKind::kBlock, 0};
}

// One launch over n rows (n <= kRowsPerLaunch).
hipError_t launch_sm_rows(hipStream_t s, const SmPlan& p, long long n, long long cols, const float* in, float* out,
                          int guard) {
  const int c = (int)cols;
  switch (p.kind) {
    case SmKind::kWave: {
      const dim3 grid((unsigned)((n + 3) / 4)), block(256);
      switch (p.sel) {
        case 1: hipLaunchKernelGGL(softmax_rows_wave<1>, grid, block, 0, s, in, out, n, c, guard); break;
        case 2: hipLaunchKernelGGL(softmax_rows_wave<2>, grid, block, 0, s, in, out, n, c, guard); break;
        case 4: hipLaunchKernelGGL(softmax_rows_wave<4>, grid, block, 0, s, in, out, n, c, guard); break;
        case 8: hipLaunchKernelGGL(softmax_rows_wave<8>, grid, block, 0, s, in, out, n, c, guard); break;
        default: hipLaunchKernelGGL(softmax_rows_wave<16>, grid, block, 0, s, in, out, n, c, guard); break;
      }
      break;
    }
    case SmKind::kWg: {
      const dim3 grid((unsigned)n), block(256);
      switch (p.sel) {
        case 8: hipLaunchKernelGGL((softmax_rows_wg<8, 256>), grid, block, 0, s, in, out, c, guard); break;
        case 16: hipLaunchKernelGGL((softmax_rows_wg<16, 256>), grid, block, 0, s, in, out, c, guard); break;
        case 32: hipLaunchKernelGGL((softmax_rows_wg<32, 256>), grid, block, 0, s, in, out, c, guard); break;
        default: hipLaunchKernelGGL((softmax_rows_wg<16, 1024>), grid, dim3(1024), 0, s, in, out, c, guard); break;
      }
      break;
    }
    case SmKind::kWgs: {
      const dim3 grid((unsigned)n);
      switch (p.sel) {
        case 40256: hipLaunchKernelGGL((softmax_rows_wgs<4, 256>), grid, dim3(256), 0, s, in, out, c, guard); break;
        case 160256: hipLaunchKernelGGL((softmax_rows_wgs<16, 256>), grid, dim3(256), 0, s, in, out, c, guard); break;
        case 161024: hipLaunchKernelGGL((softmax_rows_wgs<16, 1024>), grid, dim3(1024), 0, s, in, out, c, guard); break;
        default: hipLaunchKernelGGL((softmax_rows_wgs<32, 1024>), grid, dim3(1024), 0, s, in, out, c, guard); break;
      }
      break;
    }
    default:
      hipLaunchKernelGGL(softmax_rows_block, dim3((unsigned)n), dim3(256), 0, s, in, out, n, cols, guard);
      break;
  }
  return hipGetLastError();
}

}  // namespace

namespace bch {

const char* softmax_kernel_name(long long rows, long long cols, const float* in, const float* out) {
  if (split_plan(rows, cols).splits > 1) return "softmax_split_write";
  const SmPlan p = sm_plan(cols, in, out);
  switch (p.kind) {
    case SmKind::kWave:
      switch (p.sel) {
        case 1: return "softmax_rows_wave<1>";
        case 2: return "softmax_rows_wave<2>";
        case 4: return "softmax_rows_wave<4>";
        case 8: return "softmax_rows_wave<8>";
        default: return "softmax_rows_wave<16>";
      }
    case SmKind::kWg:
      switch (p.sel) {
        case 8: return "softmax_rows_wg<8>";
        case 16: return "softmax_rows_wg<16>";
        case 32: return "softmax_rows_wg<32>";
        default: return "softmax_rows_wg<16, 1024>";
      }
    case SmKind::kWgs:
      switch (p.sel) {
        case 40256: return "softmax_rows_wgs<4, 256>";
        case 160256: return "softmax_rows_wgs<16, 256>";
        case 161024: return "softmax_rows_wgs<16, 1024>";
        default: return "softmax_rows_wgs<32, 1024>";
      }
    default:
      return "softmax_rows_block";
  }
}

hipError_t launch_softmax_rows(hipStream_t s, long long rows, long long cols,
                               const float* in, float* out, void* ws,
                               size_t ws_bytes, bool guard) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const SplitPlan sp = split_plan(rows, cols);
  if (sp.splits > 1) {
    if (!ws || ws_bytes < softmax_workspace_bytes(rows, cols) || rows > 65535)
      return hipErrorInvalidValue;
    float* part = static_cast<float*>(ws);
    const bool vec = (cols % 4) == 0 && (reinterpret_cast<uintptr_t>(in) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    dim3 grid((unsigned)sp.splits, (unsigned)rows), block(256);
    if (vec) {
      hipLaunchKernelGGL(softmax_split_stats<true>, grid, block, 0, s, in, cols, sp.chunk, part);
      hipLaunchKernelGGL(softmax_split_write<true>, grid, block, 0, s, in, out, cols, sp.chunk, part, guard);
    } else {
      hipLaunchKernelGGL(softmax_split_stats<false>, grid, block, 0, s, in, cols, sp.chunk, part);
      hipLaunchKernelGGL(softmax_split_write<false>, grid, block, 0, s, in, out, cols, sp.chunk, part, guard);
    }
    return hipGetLastError();
  }
  const SmPlan p = sm_plan(cols, in, out);
  // rows in launches of at most kRowsPerLaunch (grids below 2^32 threads); a
  // chunk starts a whole number of rows in, which keeps the alignment the
  // float4 kernels were chosen for
  for (long long r0 = 0; r0 < rows; r0 += kRowsPerLaunch) {
    const long long n = rows - r0 < kRowsPerLaunch ? rows - r0 : kRowsPerLaunch;
    const hipError_t e = launch_sm_rows(s, p, n, cols, in + r0 * cols, out + r0 * cols, guard);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool softmax_rows_scaled_supported(long long cols, const float* in, const float* out) {
  return wave_path(cols, in, out);
}

hipError_t launch_softmax_rows_scaled(hipStream_t s, long long rows, long long cols, const float* in, float* out,
                                      float scale, int causal, int m, int r0) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (!wave_path(cols, in, out) || m < 1) return hipErrorInvalidValue;
  const int c = (int)cols;
  for (long long b = 0; b < rows; b += kRowsPerLaunch) {
    const long long n = rows - b < kRowsPerLaunch ? rows - b : kRowsPerLaunch;
    const dim3 grid((unsigned)((n + 3) / 4)), block(256);
    const float* i0 = in + b * cols;
    float* o0 = out + b * cols;
    switch (pick_nv(cols)) {
      case 1: hipLaunchKernelGGL(softmax_rows_wave_scaled<1>, grid, block, 0, s, i0, o0, n, c, scale, causal, m, b, r0); break;
      case 2: hipLaunchKernelGGL(softmax_rows_wave_scaled<2>, grid, block, 0, s, i0, o0, n, c, scale, causal, m, b, r0); break;
      case 4: hipLaunchKernelGGL(softmax_rows_wave_scaled<4>, grid, block, 0, s, i0, o0, n, c, scale, causal, m, b, r0); break;
      case 8: hipLaunchKernelGGL(softmax_rows_wave_scaled<8>, grid, block, 0, s, i0, o0, n, c, scale, causal, m, b, r0); break;
      default: hipLaunchKernelGGL(softmax_rows_wave_scaled<16>, grid, block, 0, s, i0, o0, n, c, scale, causal, m, b, r0); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_softmax_axis(hipStream_t s, long long outer, long long axis,
                               long long inner, const float* in, float* out,
                               void* ws, size_t ws_bytes, bool guard) {
  if (outer <= 0 || axis <= 0 || inner <= 0) return hipSuccess;
  if (inner == 1) return launch_softmax_rows(s, outer, axis, in, out, ws, ws_bytes, guard);
  const WidePlan wp = wide_plan(outer, axis, inner);
  if (wp.on && vec_aligned(in, out)) {
    if (ws == nullptr || ws_bytes < wide_bytes(outer, inner, wp)) return hipErrorInvalidValue;
    return launch_cols_wide(s, wp, outer, axis, inner, in, out, ws, guard);
  }
  const VecPlan vp = vec_plan(outer, axis, inner);
  if (vp.w && vec_aligned(in, out)) {
    float4* part = nullptr;
    if (vp.nchunks > 1) {
      if (ws == nullptr || ws_bytes < sizeof(float) * 2 * (size_t)(outer * vp.nchunks * inner)) return hipErrorInvalidValue;
      part = static_cast<float4*>(ws);
    }
    switch (vp.w) {
      case 1: launch_cols_vec_w<1, 256>(s, vp, outer, axis, inner / 4, in, out, part, guard); break;
      case 2: launch_cols_vec_w<2, 256>(s, vp, outer, axis, inner / 4, in, out, part, guard); break;
      case 4: launch_cols_vec_w<4, 256>(s, vp, outer, axis, inner / 4, in, out, part, guard); break;
      default: launch_cols_vec_w<8, 512>(s, vp, outer, axis, inner / 4, in, out, part, guard); break;
    }
    return hipGetLastError();
  }
  const ColPlan p = col_plan(outer, axis, inner);
  const long long blocks = outer * p.nchunks * p.strips;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  if (p.nchunks == 1) {
    hipLaunchKernelGGL(softmax_cols<true>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, axis, inner, p.cw,
                       p.strips, 1, p.rpc, nullptr, guard);
    return hipGetLastError();
  }
  const size_t need = sizeof(float) * 2 * (size_t)outer * p.nchunks * (size_t)inner;
  if (ws == nullptr || ws_bytes < need) return hipErrorInvalidValue;
  float* part = static_cast<float*>(ws);
  hipLaunchKernelGGL(softmax_cols<false>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, axis, inner, p.cw,
                     p.strips, p.nchunks, p.rpc, part, guard);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(softmax_cols_write, dim3((unsigned)blocks), dim3(256), 0, s, in, out, axis, inner, p.cw,
                     p.strips, p.nchunks, p.rpc, part, guard);
  return hipGetLastError();
}

}  // namespace bch

// Unmangled entry for the code-object path (bch_launch_code_object): the
// cols == 2048 register-resident row softmax, 4 rows per 256-thread block.
extern "C" __global__ __launch_bounds__(256) void bch_softmax_rows_2048(
    const float* in, float* out, long long rows) {
  softmax_rows_wave_body<8>(in, out, rows, 2048, 0);
}
