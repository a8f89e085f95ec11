/*
 * barracuda_hip.h -- C ABI of libbarracuda_hip.so, the MI355X (gfx950)
 * implementation of barraCuda's dense ML-ops hot path: f32 matmul and
 * batched matmul, row softmax, scaled-dot-product attention forward.
 *
 * Plain C: pointers, sizes, status codes.  No C++ or torch types cross this
 * boundary.  Every call returns a bch_status (BCH_OK == 0) and never aborts;
 * the message of the last failure is kept per context (bch_last_error) and
 * per thread for calls that fail before a context exists.
 *
 * Conventions
 *   - Matrices are row-major f32.  Device pointers come from bch_alloc (or
 *     any hipMalloc'd memory of the same device).
 *   - A context owns one HIP stream.  Compute calls enqueue on it and return
 *     without waiting; bch_download and bch_sync wait.  A context is not
 *     re-entrant: callers serialise use of one context (the Rust side holds
 *     it behind a Mutex), or use one context per thread.
 *   - Shapes are validated before anything touches the device, so a shape
 *     error is reported identically with or without a GPU.
 *
 * Each entry point names the reference interface it replaces
 * (ecoPrimals/barraCuda, paths relative to crates/barracuda/src/).
 */
#ifndef BARRACUDA_HIP_H
#define BARRACUDA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Map 1:1 onto BarracudaError (error.rs:14-130). */
typedef int bch_status;
#define BCH_OK            0
#define BCH_E_INVALID     1 /* null pointer / bad argument -> InvalidInput     (error.rs:187) */
#define BCH_E_SHAPE       2 /* inconsistent dimensions     -> ShapeMismatch/InvalidOperation (error.rs:238,243) */
#define BCH_E_NO_DEVICE   3 /* no HIP device               -> DeviceNotAvailable */
#define BCH_E_OOM         4 /* device allocation failed    -> OutOfMemory */
#define BCH_E_MODULE      5 /* code object missing/corrupt -> Device(String)   (error.rs:220) */
#define BCH_E_LAUNCH      6 /* launch rejected (resources, configuration) -> ExecutionError (error.rs:230) */
#define BCH_E_DEVICE      7 /* other HIP runtime failure   -> Device(String)   (error.rs:220) */
#define BCH_E_UNSUPPORTED 8 /* op/entry not provided       -> UnsupportedOperation */
#define BCH_E_DEVICE_LOST 9 /* the context can run no more work: a kernel
                             * faulted (memory fault, trap, assert, watchdog),
                             * an uncorrectable ECC error, or the context is
                             * gone.  Sticky: every later call on the context
                             * that touches the device returns it too.  HIP
                             * graphs captured on the context's stream are
                             * to be discarded with it (a replay would not
                             * go through the library's checks).
                             *                             -> DeviceLost(String) (error.rs:59) */

typedef struct bch_ctx bch_ctx;
typedef struct bch_event bch_event;

/* ---- context and memory: replaces the WgpuDevice side of GpuBackend
 *      (device/backend.rs:244-444; wgpu_backend.rs:122-155 download) ---- */

/* Number of visible HIP devices; BCH_E_NO_DEVICE (and *count = 0) if none. */
bch_status bch_device_count(int *count);

/* Create a context on `device` (its own stream).  code_object_dir (nullable)
 * is the directory bch_launch_code_object resolves relative names against;
 * NULL means the directory of libbarracuda_hip.so.  Env
 * BARRACUDA_HIP_DEVICE overrides device when device < 0. */
bch_status bch_ctx_create(int device, const char *code_object_dir, bch_ctx **out);
void bch_ctx_destroy(bch_ctx *ctx);

/* *lost = 1 once a call on ctx has returned BCH_E_DEVICE_LOST, else 0.
 * Replaces GpuBackend::is_lost (device/backend.rs:256), which reads the flag
 * that WgpuDevice::poll_safe sets on a device-lost panic
 * (device/wgpu_device/submission.rs:23-71).  The caller recovers with a fresh
 * context (the reference retries on a fresh device, error.rs:52-58).
 * Env BARRACUDA_HIP_INJECT_HIP_ERROR=<hipError_t value>, read by
 * bch_ctx_create, makes the context's first device call report that HIP
 * error (fault injection for this mapping; no kernel runs). */
bch_status bch_ctx_is_lost(const bch_ctx *ctx, int *lost);

/* *stream = the context's HIP stream (a hipStream_t).  No counterpart in
 * the reference, whose wgpu queue is internal: it is for callers that order
 * the context's work against their own streams or capture it into a HIP
 * graph.  Capture only calls whose workspace already exists (make each call
 * once outside the capture first, or bch_ctx_reserve): a call that would
 * have to grow the workspace while the stream is being captured fails with
 * BCH_E_UNSUPPORTED and enqueues nothing.  Once a capture has been seen on
 * the context, a later eager call that grows the workspace keeps the old
 * one alive (captured graphs still read it) until bch_ctx_destroy.  Every
 * captured call replays correctly any number of times; replays and eager
 * calls on one context must not overlap (they share the workspace). */
bch_status bch_ctx_stream(const bch_ctx *ctx, void **stream);

/* Grow the context's workspace to at least `bytes` now (outside any
 * capture), so that later calls -- captured or not -- need no allocation.
 * *bytes = the workspace's current size (0 for a fresh context).  No
 * counterpart in the reference (its buffer pool is internal); for callers
 * that capture the context's work or must not allocate in a hot loop. */
bch_status bch_ctx_reserve(bch_ctx *ctx, size_t bytes);
bch_status bch_ctx_workspace_bytes(const bch_ctx *ctx, size_t *bytes);

/* Message of the last failed call on ctx; with ctx == NULL, the calling
 * thread's last failure.  Never NULL ("" when none). */
const char *bch_last_error(const bch_ctx *ctx);
const char *bch_status_string(bch_status s);

/* backend.rs alloc_buffer / alloc_buffer_init / upload / download.
 * bch_alloc of 0 bytes returns a NULL pointer and BCH_OK.  Env
 * BARRACUDA_HIP_FAIL_ALLOC=1 makes every bch_alloc fail with BCH_E_OOM
 * (fault injection for OutOfMemory handling).
 * Like the reference's buffer pool (device/tensor_context/pool.rs:268-334),
 * bch_free keeps the block for the context's next bch_alloc of the same
 * size class (powers of two from 256 bytes to 64 MiB, then multiples of
 * 2 MiB) and returns without waiting: work queued on ctx that still reads
 * it runs before anything queued after its reuse.  Work on other streams
 * that reads a block must be complete before the block is freed.  Parked
 * blocks are released when an allocation would otherwise fail, beyond
 * BARRACUDA_HIP_POOL_MAX_MB (default 8192) of them, and by
 * bch_ctx_destroy.  Memory that bch_alloc did not hand out is freed after
 * ctx's queued work, as before. */
bch_status bch_alloc(bch_ctx *ctx, size_t bytes, void **dptr);
bch_status bch_free(bch_ctx *ctx, void *dptr);
bch_status bch_upload(bch_ctx *ctx, void *dst, const void *src, size_t bytes);
bch_status bch_download(bch_ctx *ctx, void *dst, const void *src, size_t bytes);
bch_status bch_memset(bch_ctx *ctx, void *dst, int value, size_t bytes);
/* Device-to-device copy on ctx's stream (no counterpart in GpuBackend, which
 * copies through upload/download; here it is also the known-traffic kernel
 * that calibrates the HBM byte counters used to profile the hot path). */
bch_status bch_copy(bch_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Wait for all work queued on ctx's stream (submit_and_poll, wgpu_device/
 * submission.rs:143). */
bch_status bch_sync(bch_ctx *ctx);

/* ---- hot-path compute ---- */

/* C[m,n] = A[m,k] . B[k,n], row-major, leading dimensions in elements
 * (lda >= k, ldb >= n, ldc >= n).  m, n, k >= 0; k == 0 writes zeros.
 * Replaces MatMul::execute (ops/matmul.rs:89-214: kernels K1
 * matmul_gpu_evolved_f64.wgsl, K2 matmul_cpu_tiled_f64.wgsl, K3
 * matmul_tiled_f64.wgsl) and MatmulTiled::execute (ops/matmul_tiled.rs:
 * 62-122).  Routes m <= 32 (decode shapes) to the skinny HBM-streaming
 * kernels, 32 < m <= 64 with K % 4 == 0 and 16-byte aligned A to their
 * two-block form, and everything else to the FP32-MFMA tiled kernel (64x64
 * tiles, or a split over k, when the tiles fill less than one round of the
 * CUs, whichever is modelled faster; whole rounds
 * plus k-sliced leftover tiles when the last round would be part-filled; or
 * whole rounds of 256x256 tiles on the first rows or columns of C and the
 * rest planned on its own, where that is modelled faster). */
bch_status bch_sgemm(bch_ctx *ctx, int m, int n, int k,
                     const float *A, int lda, const float *B, int ldb,
                     float *C, int ldc);

/* bch_sgemm without any device allocation: no hipMalloc, hipFree or
 * allocating library call on any path.  No counterpart in the reference; it
 * is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  The decode-shaped
 * (m <= 32) path's split-k partials go to a fixed 16 MiB device array
 * (one per GPU, held until the process ends) instead of the context's
 * workspace; shapes needing more return BCH_E_UNSUPPORTED (e.g. m = 32 with
 * n above ~65000).  The tiled kernel's split-k and leftover-tile partials
 * use the same array where they fit; otherwise the call takes fewer k
 * slices or whole tiles, as 32 < m <= 64 takes the tiles when its skinny
 * partials do not fit.  No kernel relies on the array's earlier contents.
 * Every call on one GPU shares that GPU's array, so calls that overlap in
 * time on one GPU (two contexts or streams) race: serialise them.  Results
 * are bit-identical to bch_sgemm's where both calls take the same kernels,
 * and within the f32 tolerance where this one takes fewer slices or whole
 * tiles. */
bch_status bch_sgemm_noalloc(bch_ctx *ctx, int m, int n, int k,
                             const float *A, int lda, const float *B, int ldb,
                             float *C, int ldc);

/* Activation of bch_sgemm_ex's epilogue. */
#define BCH_ACT_NONE 0
#define BCH_ACT_RELU 1 /* max(x, 0): shaders/activation/relu_f64.wgsl */
#define BCH_ACT_GELU 2 /* 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))):
                        * shaders/activation/gelu_f64.wgsl (run in f32 with
                        * WGSL's tanh); large |x| gives x (or -0) */

/* The linear layer: C = act(A . op(B) + bias), row-major, where op(B) = B
 * for transb == 0 (B [k, n], ldb >= n) and B^T for transb == 1 (B [n, k],
 * ldb >= k: the weight layout [out_features, in_features] of
 * shaders/misc/linear_f64.wgsl, y = x W^T + b).  bias (nullable) has n
 * entries and is added after the dot product, as linear_f64.wgsl does; act
 * is BCH_ACT_NONE, BCH_ACT_RELU or BCH_ACT_GELU.  Everything happens in the
 * GEMM's own epilogue: one launch per layer where the reference's
 * nn::fused_mlp (nn/fused_mlp.rs:38-168) dispatches linear_f64.wgsl and
 * then relu_f64.wgsl (gelu_f64.wgsl, ops/gelu_wgsl.rs) over the output.  transb == 0, act == NONE, bias == NULL is
 * bch_sgemm. */
bch_status bch_sgemm_ex(bch_ctx *ctx, int transb, int m, int n, int k,
                        const float *A, int lda, const float *B, int ldb,
                        const float *bias, int act, float *C, int ldc);

/* C[b] = A[b] . B[b] for b < batch; A[b] starts at A + b*strideA (elements),
 * leading dimensions k, n, n.  Replaces BatchMatMul::execute
 * (ops/batch_matmul.rs:47-144, kernel K5 batch_matmul_f64.wgsl). */
bch_status bch_sgemm_strided_batched(bch_ctx *ctx, int batch, int m, int n,
                                     int k, const float *A, long long strideA,
                                     const float *B, long long strideB,
                                     float *C, long long strideC);

/* f64 GEMM on the FP64 matrix cores, batched:
 *   C[b] = alpha * op(A[b]) * op(B[b])          (beta == 0: C is not read)
 *   C[b] = alpha * op(A[b]) * op(B[b]) + beta * C[b]   (beta != 0)
 * op(A) = A stored [m][k] (lda >= k) when transa == 0, A^T of A stored
 * [k][m] (lda >= m) when transa == 1; op(B) = B [k][n] (ldb >= n) or B^T
 * of B stored [n][k] (ldb >= k).  C [m][n], ldc >= n.  Batch b's matrices
 * start at A + b*strideA, B + b*strideB, C + b*strideC (elements).
 * Replaces GemmF64::execute / execute_gemm / execute_gemm_ex and
 * GemmCachedF64::{multiply, execute_to_buffer} (ops/linalg/gemm_f64.rs:
 * 77-456, shaders/linalg/gemm_f64.wgsl), whose buffers are packed:
 * strides m*k, k*n, m*n. */
bch_status bch_dgemm(bch_ctx *ctx, int transa, int transb, int batch, int m,
                     int n, int k, double alpha, const double *A, int lda,
                     long long strideA, const double *B, int ldb,
                     long long strideB, double beta, double *C, int ldc,
                     long long strideC);

/* Row-wise numerically stable softmax: out[r,:] = exp(x - max_r) / sum.
 * rows, cols >= 1; in == out is allowed.  Replaces the attention row
 * softmax K7 (shaders/activation/attention_softmax_f64.wgsl:24-58) and,
 * with rows == 1, the global Softmax::execute (ops/softmax.rs:58-133, K11
 * softmax_simple_f64.wgsl), which divide by the sum whatever it is: a row
 * holding NaN or +inf, or nothing but -inf, comes out all NaN.  For
 * Tensor::softmax_dim over the last axis use bch_softmax_axis with
 * inner == 1 (the same kernels, with softmax_dim's handling of such rows). */
bch_status bch_softmax_rows(bch_ctx *ctx, long long rows, long long cols,
                            const float *in, float *out);

/* Row-wise f64 softmax: out[r,:] = exp(x - m_r) / sum_j exp(x_j - m_r), m_r
 * the row maximum folded from -inf with f64::max (NaN entries skipped).
 * rows, cols >= 1 (any row count: long row counts run in several launches);
 * in == out is allowed.  Replaces the row
 * softmax of the ml.attention handler (barracuda-core/src/ipc/methods/ml/
 * forward.rs:130-140), the step between its two products (which run on
 * bch_dgemm). */
bch_status bch_softmax_rows_f64(bch_ctx *ctx, long long rows, long long cols,
                                const double *in, double *out);

/* Element-wise ops of TensorSession over n f32 elements:
 *   BCH_EW_ADD out = a + b      BCH_EW_SUB out = a - b     BCH_EW_MUL out = a * b
 *   BCH_EW_NEG out = -a         BCH_EW_FMA out = fma(a, b, c)
 *   BCH_EW_SCALE out = a * scalar
 *   BCH_EW_RELU out = max(a, 0) BCH_EW_GELU out = GELU(a) (as BCH_ACT_GELU)
 * b is read by add/sub/mul/fma, c by fma only (others may be NULL); out may
 * equal a, b or c.  Replaces the session's inline add/sub/mul/negate/fma/
 * scale shaders (session/pipelines.rs:76-145, dispatch.rs) and its ReLU and
 * GELU ops (session/mod.rs:340-359: ops/relu.rs, ops/gelu_wgsl.rs). */
#define BCH_EW_ADD 0
#define BCH_EW_SUB 1
#define BCH_EW_MUL 2
#define BCH_EW_NEG 3
#define BCH_EW_FMA 4
#define BCH_EW_SCALE 5
#define BCH_EW_RELU 6
#define BCH_EW_GELU 7
bch_status bch_elementwise(bch_ctx *ctx, int op, long long n, const float *a,
                           const float *b, const float *c, float scalar,
                           float *out);

/* Layer normalisation of each row of a [rows, cols] f32 matrix:
 *   out = (x - mean) / sqrt(var + eps), mean and (biased) var over the row.
 * No affine parameters; in == out is allowed; any row count (long row
 * counts run in several launches).  Replaces
 * TensorSession::layer_norm (session/mod.rs:379-398, epsilon 1e-5 at
 * dispatch.rs:221-240) and LayerNorm::execute / Tensor::layer_norm_wgsl
 * (ops/layer_norm_wgsl.rs, shaders/norm/layer_norm_f64.wgsl). */
bch_status bch_layer_norm(bch_ctx *ctx, long long rows, long long cols,
                          float eps, const float *in, float *out);

/* Multi-head layout changes of TensorSession (session/mod.rs:423-480):
 *   bch_head_split:  in [B, S, H*D] -> out [B, H, S, D]
 *                    (out[b][h][s][d] = in[b][s][h*D + d],
 *                    shaders/tensor/head_split_f64.wgsl)
 *   bch_head_concat: in [B, H, S, D] -> out [B, S, H*D]
 *                    (the inverse map, head_concat_f64.wgsl)
 * Dense f32 buffers; in and out must not overlap (BCH_E_INVALID when
 * in == out).  Bit-exact copies (HBM-streaming, 8 bytes per element).
 * Dimensions >= 1; B*S*H*D*4 bytes each. */
bch_status bch_head_split(bch_ctx *ctx, int B, int S, int H, int D,
                          const float *in, float *out);
bch_status bch_head_concat(bch_ctx *ctx, int B, int S, int H, int D,
                           const float *in, float *out);

/* Softmax along a middle axis of a tensor viewed as [outer, axis, inner]
 * (element (o,j,i) at (o*axis + j)*inner + i).  inner == 1 is the row case.
 * Replaces Tensor::softmax_dim (ops/tensor_axis_ops.rs:67-126) for any
 * axis, with its host loop's handling of a slice whose sum is not > 0
 * (one holding NaN or +inf, or nothing but -inf): the slice keeps its
 * exp(x - max) un-normalised (:108-114, `if sum > 0.0`).  A long axis on
 * few columns is cut into chunks whose per-column (max, sum) states use the
 * context's workspace (grown on demand); in == out is allowed. */
bch_status bch_softmax_axis(bch_ctx *ctx, long long outer, long long axis,
                            long long inner, const float *in, float *out);

/* Fused scaled-dot-product attention forward, [B,H,S,D] row-major:
 *   o[b,h,i,:] = sum_j softmax_j(scale * q_i . k_j) v_j
 * with j <= i when causal (causal requires Sq == Skv, as the reference's
 * causal ops take one seq_len).  Non-causal Sq may differ from Skv
 * (cross-attention).  Any D >= 1, as the reference's ops take: up to
 * D = 256 one fused kernel that never materialises the Sq x Skv score
 * matrix and uses no scratch; above D = 256 the scores of one chunk of
 * query rows at a time (at most 256 MiB) go through the context's
 * workspace (grown on demand, like the GEMM's) in three steps -- Q K^T,
 * scaled and masked row softmax, P V -- on the MFMA GEMM.  Replaces Attention::execute (ops/attention/
 * compute.rs:21-111: K6 attention_matmul_f64.wgsl -> K7 -> K9
 * attention_apply_f64.wgsl), ScaledDotProductAttention (ops/
 * scaled_dot_product_attention/compute.rs:19-108), CausalAttention (ops/
 * causal_attn/compute.rs:24-115, K8 causal_attention_softmax_f64.wgsl),
 * the CPU causal_attention (ops/causal_attention.rs:52-134) and
 * FlashAttention::execute (ops/flash_attention.rs:96-145, K13). */
bch_status bch_sdpa_fwd(bch_ctx *ctx, int B, int H, int Sq, int Skv, int D,
                        float scale, int causal, const float *q,
                        const float *k, const float *v, float *o);

/* Layout of one attention operand: element (b, h, i, d) is at
 * b*batch_stride + h*head_stride + i*row_stride + d (elements; the head
 * dimension is contiguous).  Dense [B,H,S,D] is {H*S*D, S*D, D}; the
 * [B,S,H*D] output of a projection GEMM viewed per head is {S*H*D, D, H*D}. */
typedef struct bch_attn_layout {
  long long batch_stride;
  long long head_stride;
  long long row_stride;
} bch_attn_layout;

/* bch_sdpa_fwd over strided operands, with Hkv key/value heads shared by
 * the H query heads (query head h reads key/value head h / (H / Hkv);
 * H % Hkv == 0, else BCH_E_INVALID "num_q_heads (H) must be divisible by
 * num_kv_heads (Hkv)").  q, o have H heads and Sq rows; k, v have Hkv heads
 * and Skv rows.  Strides >= 0, row_stride >= D (and below 2^31 when
 * D > 256).  Replaces
 * GroupedQueryAttention::execute (ops/grouped_query_attention/compute.rs:
 * 27-121: gqa_matmul_f64.wgsl -> gqa_softmax_f64.wgsl -> gqa_apply_f64.wgsl;
 * validation mod.rs:84-147) with Hkv < H, and the attention core of
 * MultiHeadAttention::execute (ops/mha/mod.rs:152-187) together with its
 * head_split / head_concat copies (ops/mha/projections.rs:18-58,
 * shaders/tensor/head_split_f64.wgsl, head_concat_f64.wgsl), which become
 * the strides of the [B,S,H*D] projection buffers. */
bch_status bch_sdpa_fwd_ex(bch_ctx *ctx, int B, int H, int Hkv, int Sq,
                           int Skv, int D, float scale, int causal,
                           const float *q, bch_attn_layout q_layout,
                           const float *k, bch_attn_layout k_layout,
                           const float *v, bch_attn_layout v_layout,
                           float *o, bch_attn_layout o_layout);

/* ---- seeded synthetic inputs, generated in HBM ---- */

/* Fill dst[0..n) from the reference's seeded generators: uniform [lo, hi)
 * from the Knuth LCG of rng.rs:20-70 (increment 1, u = (state >> 11) 2^-53,
 * x = lo + (hi - lo) u), normal from ops/lattice/constants.rs:11-49 (MMIX
 * increment, Box-Muller with u1 guarded by 1e-30, x = mu + sigma g, two
 * draws per element).  Element i equals a sequential host fill.  *state is
 * the generator state before the fill and is advanced past it (n steps, 2n
 * for normal), so successive fills continue one stream, as the reference
 * fills tensors in argument order.  Device counterpart of the seeded
 * constructors Tensor::rand_with_rng / randn_with_rng (tensor/ops.rs:79-125). */
bch_status bch_fill_uniform(bch_ctx *ctx, float *dst, size_t n,
                            unsigned long long *state, double lo, double hi);
bch_status bch_fill_normal(bch_ctx *ctx, float *dst, size_t n,
                           unsigned long long *state, double mu, double sigma);

/* ---- precompiled code objects: GpuBackend::dispatch_binary
 *      (device/backend.rs:344-354) ---- */

/* Load (and cache per context) a gfx950 code object and launch `entry` on
 * grid[3] workgroups of block[3] threads.  args/nargs: kernelParams as in
 * hipModuleLaunchKernel (args[i] points at the i-th argument's value).
 * code_object is either an in-memory image (len > 0) or, with len == 0, a
 * NUL-terminated path (relative paths resolve against code_object_dir). */
bch_status bch_launch_code_object(bch_ctx *ctx, const void *code_object,
                                  size_t len, const char *entry,
                                  const unsigned grid[3],
                                  const unsigned block[3], void **args,
                                  size_t nargs, size_t shared_bytes);

/* ---- timing on the context's stream (the hot path's own launches) ---- */
bch_status bch_event_create(bch_ctx *ctx, bch_event **ev);
bch_status bch_event_record(bch_ctx *ctx, bch_event *ev);
/* Elapsed milliseconds between two recorded events (waits for `stop`). */
bch_status bch_event_elapsed_ms(bch_event *start, bch_event *stop, float *ms);
void bch_event_destroy(bch_event *ev);

/* Name of the kernel a bch_sgemm / bch_layer_norm / bch_softmax_rows_f64
 * call of this shape (and, for layer norm and the f64 softmax, these
 * buffers: their 16-byte alignment picks the kernel) launches, for
 * profilers and tests. */
const char *bch_sgemm_kernel_name(int m, int n, int k);
const char *bch_layer_norm_kernel_name(long long rows, long long cols,
                                       const float *in, const float *out);
const char *bch_softmax_rows_f64_kernel_name(long long rows, long long cols,
                                             const double *in,
                                             const double *out);

#ifdef __cplusplus
}
#endif

#endif /* BARRACUDA_HIP_H */
