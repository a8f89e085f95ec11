/*
 * bc_oracle.c -- CPU oracle for the barraCuda dense ML-ops hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (barracuda_amd/) links,
 * loads or calls this file.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker / the timed
 * CPU baseline, never as the thing measured or shipped.
 *
 * Reference: ecoPrimals/barraCuda (Rust + WGSL), which cannot be compiled in
 * this image (no cargo/rustc, dependencies not vendored), so every function
 * here is a C restatement of the reference's algorithm, citing the file:line
 * it follows.  Paths are relative to crates/barracuda/src/ of the reference.
 *
 * Three families:
 *   1. seeded input generators        (rng.rs, ops/lattice/constants.rs)
 *   2. f64 oracles (ground truth)     (the mathematical contract of each op)
 *   3. f32 restatements that follow the reference's own accumulation order
 *      (the CPU paths verbatim, the WGSL shaders as evaluated in f32 after
 *      shaders/precision/compiler.rs:91-109 downcasts them).
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   generators        -- recurrence restated independently in Python with
 *                        exact u64 arithmetic; jump-ahead vs stepping;
 *                        moment tests as in ops/lattice/constants.rs tests.
 *   f64 oracles       -- literal vectors from the reference tests (golden
 *                        fixtures under tests/golden/), closed forms
 *                        (uniform scores -> mean of V, single key -> V row,
 *                        causal row 0 -> V[0]), brute force on tiny shapes
 *                        against numpy float64 / longdouble.
 *   f32 restatements  -- agreement with the f64 oracle to the reference's
 *                        tolerances, exactness on integer-valued inputs, and
 *                        order-sensitivity probes that a transposed operand
 *                        or dropped term fails.
 *   inline handlers   -- (the f64 ml.attention and
 *                        tensor.matmul_inline handlers) the handler tests' vectors
 *                        (ml_tests.rs:128-165, sprint56b_tests.rs:618-669),
 *                        closed forms (one key -> its V row, equal scores ->
 *                        the mean of V, the one-hot case), numpy longdouble
 *                        brute force, and planted mistakes (no scale, V
 *                        transposed, max not subtracted) that must fail.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -shared).  -ffp-contract=off so
 * that every fused multiply-add here is an explicit fma()/fmaf() call that
 * mirrors a mul_add() in the reference, and nothing else is contracted.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define BCO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------
 * 1. Seeded generators
 * ---------------------------------------------------------------------- */

/* rng.rs:20 LCG_MULTIPLIER, rng.rs:28-30 lcg_step (increment 1). */
static const uint64_t LCG_MUL = 6364136223846793005ULL;
/* ops/lattice/constants.rs:14 LCG_INCREMENT (Knuth MMIX). */
static const uint64_t LCG_INC_MMIX = 1442695040888963407ULL;

/* Affine map x -> a*x + c (mod 2^64) raised to the n-th power: the state n
 * steps ahead.  Used to split a sequence across threads bit-identically. */
static void lcg_jump(uint64_t inc, uint64_t n, uint64_t *A, uint64_t *C)
{
    uint64_t acc_a = 1, acc_c = 0;       /* identity */
    uint64_t cur_a = LCG_MUL, cur_c = inc; /* one step */
    while (n) {
        if (n & 1) {                       /* acc = cur o acc */
            acc_c = cur_a * acc_c + cur_c;
            acc_a = cur_a * acc_a;
        }
        cur_c = cur_a * cur_c + cur_c;     /* cur = cur o cur */
        cur_a = cur_a * cur_a;
        n >>= 1;
    }
    *A = acc_a;
    *C = acc_c;
}

BCO_API uint64_t bco_lcg_advance(uint64_t state, uint64_t inc, uint64_t n)
{
    uint64_t a, c;
    lcg_jump(inc, n, &a, &c);
    return a * state + c;
}

/* rng.rs:54-56 state_to_f64: upper 53 bits / 2^53. */
static inline double state_to_f64(uint64_t s)
{
    return (double)(s >> 11) / 9007199254740992.0;
}

/* Uniform [lo, hi) from rng.rs:61-70 (uniform_f64_sequence: step, then
 * convert), mapped affinely: x = lo + (hi - lo) * u.  With lo=-1, hi=1 this
 * is the 2u - 1 of the benchmark configs.  *state is advanced by n steps.
 * Evaluated in f64 and rounded once to f32. */
BCO_API void bco_fill_uniform(uint64_t *state, double lo, double hi,
                              float *out, size_t n)
{
    const uint64_t s0 = *state;
    #pragma omp parallel
    {
        size_t nt = 1, tid = 0;
#ifdef _OPENMP
        nt = (size_t)omp_get_num_threads();
        tid = (size_t)omp_get_thread_num();
#endif
        size_t chunk = (n + nt - 1) / nt;
        size_t b = tid * chunk, e = b + chunk < n ? b + chunk : n;
        if (b < e) {
            uint64_t s = bco_lcg_advance(s0, 1, (uint64_t)b);
            for (size_t i = b; i < e; ++i) {
                s = s * LCG_MUL + 1;
                out[i] = (float)(lo + (hi - lo) * state_to_f64(s));
            }
        }
    }
    *state = bco_lcg_advance(s0, 1, (uint64_t)n);
}

/* ops/lattice/constants.rs:38-49: lcg_uniform_f64 (MMIX increment) and
 * lcg_gaussian (Box-Muller, u1 guarded by 1e-30, cos branch), scaled:
 * x = mu + sigma * g.  Two draws per output; *state advances 2n steps. */
BCO_API void bco_fill_normal(uint64_t *state, double mu, double sigma,
                             float *out, size_t n)
{
    const uint64_t s0 = *state;
    const double two_pi = 2.0 * 3.14159265358979323846;
    #pragma omp parallel
    {
        size_t nt = 1, tid = 0;
#ifdef _OPENMP
        nt = (size_t)omp_get_num_threads();
        tid = (size_t)omp_get_thread_num();
#endif
        size_t chunk = (n + nt - 1) / nt;
        size_t b = tid * chunk, e = b + chunk < n ? b + chunk : n;
        if (b < e) {
            uint64_t s = bco_lcg_advance(s0, LCG_INC_MMIX, 2 * (uint64_t)b);
            for (size_t i = b; i < e; ++i) {
                s = s * LCG_MUL + LCG_INC_MMIX;
                double u1 = state_to_f64(s);
                s = s * LCG_MUL + LCG_INC_MMIX;
                double u2 = state_to_f64(s);
                double g = sqrt(-2.0 * log(u1 > 1e-30 ? u1 : 1e-30)) * cos(two_pi * u2);
                out[i] = (float)(mu + sigma * g);
            }
        }
    }
    *state = bco_lcg_advance(s0, LCG_INC_MMIX, 2 * (uint64_t)n);
}

/* ------------------------------------------------------------------------
 * 2. f64 oracles (the mathematical contract; inputs are the f32 tensors)
 * ---------------------------------------------------------------------- */

/* C = A * B, row-major, leading dimensions lda/ldb/ldc, double accumulation.
 * Contract of ops/matmul.rs:89-214 (C[m,n] = sum_p A[m,p] B[p,n]).
 * rows_sel (nullable, n_sel entries) restricts the rows computed; C then
 * holds n_sel rows, in that order.  Parallel over rows. */
BCO_API void bco_matmul_f64(int m, int n, int k, const float *A, long lda,
                            const float *B, long ldb, double *C, long ldc,
                            const int *rows_sel, int n_sel)
{
    int nrows = rows_sel ? n_sel : m;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int r = 0; r < nrows; ++r) {
        int i = rows_sel ? rows_sel[r] : r;
        double *c = C + (long)r * ldc;
        for (int j = 0; j < n; ++j) c[j] = 0.0;
        for (int p = 0; p < k; ++p) {
            double a = (double)A[(long)i * lda + p];
            const float *b = B + (long)p * ldb;
            for (int j = 0; j < n; ++j) c[j] += a * (double)b[j];
        }
    }
}

/* Row-wise softmax in f64: y = exp(x - max) / sum exp(x - max).
 * Contract of ops/tensor_axis_ops.rs:67-126 with axis = last. */
BCO_API void bco_softmax_rows_f64(long rows, long cols, const float *x, double *y)
{
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        double *yr = y + r * cols;
        double mx = -INFINITY;
        for (long j = 0; j < cols; ++j) if ((double)xr[j] > mx) mx = xr[j];
        double s = 0.0;
        for (long j = 0; j < cols; ++j) { yr[j] = exp((double)xr[j] - mx); s += yr[j]; }
        for (long j = 0; j < cols; ++j) yr[j] /= s;
    }
}

/* Scaled-dot-product attention in f64, [B,H,S,D] row-major contiguous:
 *   O[i] = sum_j softmax_j(scale * q_i . k_j) v_j, with j <= i when causal
 * (causal: the top-left-aligned mask of ops/causal_attention.rs:85-90).
 * Contract of ops/attention/compute.rs:21-111 (non-causal, Sq may differ
 * from Skv) and ops/causal_attention.rs:52-134 (causal, Sq == Skv).
 * heads_sel (nullable) restricts the (b*H + h) heads computed; O then holds
 * n_sel heads of [Sq, D] each, in that order.  Parallel over (head, row). */
/* One query row i of head bh: o_i = sum_j softmax_j(scale q_i.k_j) v_j over
 * j < Skv (j <= i when causal), all in double.  p: Skv doubles of scratch. */
static void sdpa_row_f64(int Sq, int Skv, int D, double scale, int causal,
                         const float *q, const float *k, const float *v,
                         int bh, int i, double *oi, double *p)
{
    const float *qi = q + ((long)bh * Sq + i) * D;
    const float *kh = k + (long)bh * Skv * D;
    const float *vh = v + (long)bh * Skv * D;
    int jend = causal ? (i + 1 < Skv ? i + 1 : Skv) : Skv;
    double mx = -INFINITY;
    for (int j = 0; j < jend; ++j) {
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)qi[d] * (double)kh[(long)j * D + d];
        p[j] = s * scale;
        if (p[j] > mx) mx = p[j];
    }
    double sum = 0.0;
    for (int j = 0; j < jend; ++j) { p[j] = exp(p[j] - mx); sum += p[j]; }
    for (int d = 0; d < D; ++d) oi[d] = 0.0;
    for (int j = 0; j < jend; ++j) {
        double w = p[j] / sum;
        const float *vj = vh + (long)j * D;
        for (int d = 0; d < D; ++d) oi[d] += w * (double)vj[d];
    }
}

BCO_API void bco_sdpa_f64(int B, int H, int Sq, int Skv, int D, double scale,
                          int causal, const float *q, const float *k,
                          const float *v, double *o, const int *heads_sel,
                          int n_sel)
{
    int nheads = heads_sel ? n_sel : B * H;
    #pragma omp parallel
    {
        double *p = (double *)malloc(sizeof(double) * (size_t)Skv);
        #pragma omp for schedule(dynamic, 4) collapse(2)
        for (int hh = 0; hh < nheads; ++hh) {
            for (int i = 0; i < Sq; ++i) {
                int bh = heads_sel ? heads_sel[hh] : hh;
                sdpa_row_f64(Sq, Skv, D, scale, causal, q, k, v, bh, i,
                             o + ((long)hh * Sq + i) * D, p);
            }
        }
        free(p);
    }
}

/* The same oracle on a row sample of every head: rows[bh * n_rows + r] is
 * the r-th query row taken from head bh (of all B*H), written to
 * o[(bh * n_rows + r) * D ..]. */
BCO_API void bco_sdpa_f64_rows(int B, int H, int Sq, int Skv, int D,
                               double scale, int causal, const float *q,
                               const float *k, const float *v, double *o,
                               const int *rows, int n_rows)
{
    int nheads = B * H;
    #pragma omp parallel
    {
        double *p = (double *)malloc(sizeof(double) * (size_t)Skv);
        #pragma omp for schedule(dynamic, 4) collapse(2)
        for (int bh = 0; bh < nheads; ++bh) {
            for (int r = 0; r < n_rows; ++r) {
                long idx = (long)bh * n_rows + r;
                sdpa_row_f64(Sq, Skv, D, scale, causal, q, k, v, bh, rows[idx], o + idx * D, p);
            }
        }
        free(p);
    }
}

/* ------------------------------------------------------------------------
 * 3. f32 restatements of the reference's own algorithms
 * ---------------------------------------------------------------------- */

/* cpu_executor/executor.rs:241-260 execute_matmul_cpu: rayon over rows of C
 * (par_chunks_mut(n)), then j, then p with sum = a.mul_add(b, sum).
 * Also the CPU-path baseline timed by bench.py (OpenMP over rows stands in
 * for rayon's row split; the per-row arithmetic is identical). */
BCO_API void bco_matmul_cpu_exec_f32(int m, int n, int k, const float *A,
                                     const float *B, float *C, int row_begin,
                                     int row_end)
{
    if (row_end > m) row_end = m;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int i = row_begin; i < row_end; ++i) {
        for (int j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (int p = 0; p < k; ++p)
                sum = fmaf(A[(long)i * k + p], B[(long)p * n + j], sum);
            C[(long)i * n + j] = sum;
        }
    }
}

/* shaders/linalg/gemm_f64.wgsl:33-91 (GemmF64, ops/linalg/gemm_f64.rs:
 * 153-249): per batch b (packed strides m*k, k*n, m*n), per (row, col),
 * acc = acc + A(row, kk) * B(kk, col) over kk in order (16-wide tiles
 * walked in order, :63-80; contracted), A(row, kk) = A[row*k + kk] or, with
 * trans_a, A[kk*m + row] (:51-56), likewise B; then C = alpha * acc, plus
 * beta * C_in when beta != 0 (:84-89).  cin may be NULL (read as zero). */
BCO_API void bco_gemm_f64_wgsl(int trans_a, int trans_b, int batch, int m,
                               int n, int k, double alpha, const double *A,
                               const double *B, double beta,
                               const double *cin, double *C)
{
    #pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < batch; ++b) {
        for (int row = 0; row < m; ++row) {
            const double *a = A + (long)b * m * k;
            const double *bb = B + (long)b * k * n;
            for (int col = 0; col < n; ++col) {
                double acc = 0.0;
                for (int kk = 0; kk < k; ++kk) {
                    const double av = trans_a ? a[(long)kk * m + row] : a[(long)row * k + kk];
                    const double bv = trans_b ? bb[(long)col * k + kk] : bb[(long)kk * n + col];
                    acc = fma(av, bv, acc);
                }
                const long ci = (long)b * m * n + (long)row * n + col;
                const double c0 = cin ? cin[ci] : 0.0;
                C[ci] = beta != 0.0 ? alpha * acc + beta * c0 : alpha * acc;
            }
        }
    }
}

/* shaders/misc/linear_f64.wgsl:21-44 in f32: y[b][o] = sum over in_f, in
 * order, of x[b][in_f] * W[o][in_f] (:34-38, sum += x * w, contracted), then
 * + bias[o] when bias != NULL (:41-43).  W is [out, in] (:17).  relu != 0
 * then applies relu_f64.wgsl (max(x, 0)) in place, as nn/fused_mlp.rs:
 * 139-151 dispatches it after every linear layer. */
BCO_API void bco_linear_f32(int batch, int in_f, int out_f, const float *X,
                            const float *W, const float *bias, int relu,
                            float *Y)
{
    #pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < batch; ++b) {
        for (int o = 0; o < out_f; ++o) {
            const float *x = X + (long)b * in_f;
            const float *w = W + (long)o * in_f;
            float sum = 0.0f;
            for (int i = 0; i < in_f; ++i) sum = fmaf(x[i], w[i], sum);
            if (bias) sum += bias[o];
            if (relu) sum = sum > 0.0f ? sum : 0.0f;
            Y[(long)b * out_f + o] = sum;
        }
    }
}

/* shaders/math/matmul_gpu_evolved_f64.wgsl:73-152 (K1) in f32: per 32-wide
 * k-tile, groups of four evaluated as a0*b0 + (a1*b1 + (a2*b2 + (a3*b3 +
 * acc))) (:124-127), then the remainder sequentially (:129-138).  The
 * driver's FMA contraction is modelled as contracting every product into
 * the sum to its right (fmaf).  K2 (matmul_cpu_tiled_f64.wgsl:140-143) has
 * the same order. */
BCO_API void bco_matmul_k1_f32(int m, int n, int k, const float *A,
                               const float *B, float *C)
{
    const int TILE = 32;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int t0 = 0; t0 < k; t0 += TILE) {
                int lim = k - t0 < TILE ? k - t0 : TILE;
                int kk = 0;
                for (; kk + 4 <= lim; kk += 4) {
                    int p = t0 + kk;
                    float a0 = A[(long)i * k + p], a1 = A[(long)i * k + p + 1];
                    float a2 = A[(long)i * k + p + 2], a3 = A[(long)i * k + p + 3];
                    float b0 = B[(long)p * n + j], b1 = B[(long)(p + 1) * n + j];
                    float b2 = B[(long)(p + 2) * n + j], b3 = B[(long)(p + 3) * n + j];
                    acc = fmaf(a0, b0, fmaf(a1, b1, fmaf(a2, b2, fmaf(a3, b3, acc))));
                }
                for (; kk < lim; ++kk) {
                    int p = t0 + kk;
                    acc = fmaf(A[(long)i * k + p], B[(long)p * n + j], acc);
                }
            }
            C[(long)i * n + j] = acc;
        }
    }
}

/* shaders/math/matmul_tiled_f64.wgsl:44-72 (K3) in f32: sequential k,
 * sum = sum + a*b (:68), contracted.  Also shaders/math/batch_matmul_f64.wgsl
 * :33-37 (K5) per batch: batch stride m*k, k*n, m*n (:30-31,39). */
BCO_API void bco_batch_matmul_seq_f32(int batch, int m, int n, int k,
                                      const float *A, const float *B, float *C)
{
    #pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int b = 0; b < batch; ++b) {
        for (int i = 0; i < m; ++i) {
            const float *a = A + (long)b * m * k + (long)i * k;
            const float *bb = B + (long)b * k * n;
            float *c = C + (long)b * m * n + (long)i * n;
            for (int j = 0; j < n; ++j) {
                float sum = 0.0f;
                for (int p = 0; p < k; ++p) sum = fmaf(a[p], bb[(long)p * n + j], sum);
                c[j] = sum;
            }
        }
    }
}

/* ops/tensor_axis_ops.rs:67-126 softmax_dim, f32, for one axis given as
 * (outer, axis, inner) with element (o, j, in) at (o*axis + j)*inner + in:
 * max from -inf updated on v > max (:91-99), exp(v - max) with a
 * sequential f32 sum (:102-110), divide only when sum > 0 (:113-119).
 * Single-threaded as in the reference (this is the CPU baseline for the
 * softmax config); rows [row_begin, row_end) of outer*inner slices. */
BCO_API void bco_softmax_dim_f32(long outer, long axis, long inner,
                                 const float *x, float *y, long slice_begin,
                                 long slice_end)
{
    long nslices = outer * inner;
    if (slice_end > nslices) slice_end = nslices;
    for (long r = slice_begin; r < slice_end; ++r) {
        long o = r / inner, in = r % inner;
        long base = o * axis * inner + in;
        float mx = -INFINITY;
        for (long j = 0; j < axis; ++j) {
            float v = x[base + j * inner];
            if (v > mx) mx = v;
        }
        float sum = 0.0f;
        for (long j = 0; j < axis; ++j) {
            float e = expf(x[base + j * inner] - mx);
            y[base + j * inner] = e;
            sum += e;
        }
        if (sum > 0.0f)
            for (long j = 0; j < axis; ++j) y[base + j * inner] /= sum;
    }
}

/* ops/softmax.rs:58-133 with shaders/activation/softmax_simple_f64.wgsl:
 * 21-51 (K11): one softmax over ALL elements (flattened), f32. */
BCO_API void bco_softmax_global_f32(long size, const float *x, float *y)
{
    bco_softmax_dim_f32(1, size, 1, x, y, 0, 1);
}

/* Three-pass attention of ops/attention/compute.rs:21-111, in f32:
 *   K6 shaders/math/attention_matmul_f64.wgsl:39-59: sequential d,
 *      score += q*k (contracted), then score / sqrt(f32(D));
 *   K7 shaders/activation/attention_softmax_f64.wgsl:37-57: max from -1e9,
 *      exp, sequential sum, divide;
 *      or, when causal, K8 causal_attention_softmax_f64.wgsl:46-72 (max from
 *      -1e10 over j <= i, masked weights 0);
 *   K9 shaders/attention/attention_apply_f64.wgsl:42-56: sequential j,
 *      sum += w*v (contracted).
 * Evaluated per (b,h) head, which is what the reference computes once its
 * 2 GiB score buffers are out of reach.  heads_sel as in bco_sdpa_f64. */
BCO_API void bco_attention_3pass_f32(int B, int H, int Sq, int Skv, int D,
                                     int causal, const float *q,
                                     const float *k, const float *v, float *o,
                                     const int *heads_sel, int n_sel)
{
    int nheads = heads_sel ? n_sel : B * H;
    float sd = sqrtf((float)D);
    #pragma omp parallel
    {
        float *w = (float *)malloc(sizeof(float) * (size_t)Skv);
        #pragma omp for schedule(dynamic, 4) collapse(2)
        for (int hh = 0; hh < nheads; ++hh) {
            for (int i = 0; i < Sq; ++i) {
                int bh = heads_sel ? heads_sel[hh] : hh;
                const float *qi = q + ((long)bh * Sq + i) * D;
                const float *kh = k + (long)bh * Skv * D;
                const float *vh = v + (long)bh * Skv * D;
                float *oi = o + ((long)hh * Sq + i) * D;
                for (int j = 0; j < Skv; ++j) {
                    float s = 0.0f;
                    for (int d = 0; d < D; ++d) s = fmaf(qi[d], kh[(long)j * D + d], s);
                    w[j] = s / sd;
                }
                if (!causal) {
                    float mx = -1e9f;
                    for (int j = 0; j < Skv; ++j) mx = fmaxf(mx, w[j]);
                    float sum = 0.0f;
                    for (int j = 0; j < Skv; ++j) { w[j] = expf(w[j] - mx); sum += w[j]; }
                    for (int j = 0; j < Skv; ++j) w[j] = w[j] / sum;
                } else {
                    float mx = -1e10f;
                    for (int j = 0; j <= i && j < Skv; ++j) mx = fmaxf(mx, w[j]);
                    float sum = 0.0f;
                    for (int j = 0; j < Skv; ++j) {
                        if (j <= i) { w[j] = expf(w[j] - mx); sum += w[j]; }
                        else w[j] = 0.0f;
                    }
                    for (int j = 0; j <= i && j < Skv; ++j) w[j] = w[j] / sum;
                }
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int j = 0; j < Skv; ++j) acc = fmaf(w[j], vh[(long)j * D + d], acc);
                    oi[d] = acc;
                }
            }
        }
        free(w);
    }
}

/* ops/causal_attention.rs:52-134 causal_attention, f32, serial:
 *   score = sum_d q.mul_add(k, score) (:89), / sqrt(D) (:69,92);
 *   max over finite scores (:96-100); exp(s - max), sequential sum, masked
 *   entries 0 (:101-109); divide every entry by sum (:110-112);
 *   out = sum_j s_j.mul_add(v, acc) over all j (:115-122).
 * Heads [head_begin, head_end) of the B*H heads (the CPU baseline times a
 * subset); O holds [B*H, S, D] and only those heads are written. */
BCO_API void bco_causal_attention_cpu_f32(int B, int H, int S, int D,
                                          const float *q, const float *k,
                                          const float *v, float *o,
                                          int head_begin, int head_end)
{
    float *sc = (float *)malloc(sizeof(float) * (size_t)S);
    float scale = sqrtf((float)D);
    if (head_end > B * H) head_end = B * H;
    for (int bh = head_begin; bh < head_end; ++bh) {
        const float *qh = q + (long)bh * S * D;
        const float *kh = k + (long)bh * S * D;
        const float *vh = v + (long)bh * S * D;
        float *oh = o + (long)bh * S * D;
        for (int i = 0; i < S; ++i) {
            for (int j = 0; j < S; ++j) sc[j] = -INFINITY;
            for (int j = 0; j <= i; ++j) {
                float s = 0.0f;
                for (int d = 0; d < D; ++d) s = fmaf(qh[(long)i * D + d], kh[(long)j * D + d], s);
                sc[j] = s / scale;
            }
            float mx = -INFINITY;
            for (int j = 0; j < S; ++j) if (isfinite(sc[j])) mx = fmaxf(mx, sc[j]);
            float sum = 0.0f;
            for (int j = 0; j < S; ++j) {
                if (isfinite(sc[j])) { sc[j] = expf(sc[j] - mx); sum += sc[j]; }
                else sc[j] = 0.0f;
            }
            for (int j = 0; j < S; ++j) sc[j] /= sum;
            for (int d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int j = 0; j < S; ++j) acc = fmaf(sc[j], vh[(long)j * D + d], acc);
                oh[(long)i * D + d] = acc;
            }
        }
    }
    free(sc);
}

/* Max of |x - ref| / max(|ref|, 1) over n elements: the scale used by
 * tolerances/mod.rs:44-54 (check), returned as a number.  Non-finite
 * entries must match exactly, otherwise the result is +inf.  Used by the
 * tests to compare multi-GB outputs without a numpy temporary. */
BCO_API double bco_max_rel_err(size_t n, const float *x, const double *ref)
{
    double worst = 0.0;
    #pragma omp parallel for reduction(max : worst) schedule(static)
    for (size_t i = 0; i < n; ++i) {
        double r = ref[i], c = (double)x[i], e;
        if (!isfinite(r) || !isfinite(c)) e = (c == r) ? 0.0 : INFINITY;
        else e = fabs(c - r) / (fabs(r) > 1.0 ? fabs(r) : 1.0);
        if (e > worst) worst = e;
    }
    return worst;
}

/* Same metric, f32 reference. */
BCO_API double bco_max_rel_err_f32ref(size_t n, const float *x, const float *ref)
{
    double worst = 0.0;
    #pragma omp parallel for reduction(max : worst) schedule(static)
    for (size_t i = 0; i < n; ++i) {
        double r = (double)ref[i], c = (double)x[i], e;
        if (!isfinite(r) || !isfinite(c)) e = (c == r) ? 0.0 : INFINITY;
        else e = fabs(c - r) / (fabs(r) > 1.0 ? fabs(r) : 1.0);
        if (e > worst) worst = e;
    }
    return worst;
}

BCO_API int bco_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Thread count of the OpenMP loops above (the CPU baselines time the
 * reference's serial paths with 1 and its rayon paths with all cores). */
BCO_API void bco_set_num_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------
 * 4. The steps either side of the path: GELU and layer norm (TensorSession
 *    session/mod.rs:349-398, dispatch.rs:196-240; the GEMM epilogue)
 * ---------------------------------------------------------------------- */

/* shaders/activation/gelu_f64.wgsl:17-31 in double:
 * 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))), libm tanh. */
BCO_API void bco_gelu_f64(size_t n, const float *x, double *y)
{
    for (size_t i = 0; i < n; ++i) {
        double v = (double)x[i];
        double x3 = v * v * v;
        double inner = 0.7978845608 * (v + 0.044715 * x3);
        y[i] = 0.5 * v * (1.0 + tanh(inner));
    }
}

/* gelu_f64.wgsl as the session runs it: downcast to f32 with tanh_f64 ->
 * the WGSL tanh builtin (shaders/precision/compiler.rs:91-109, bound at
 * session/pipelines.rs:54-62,154), same operation order. */
BCO_API void bco_gelu_wgsl_f32(size_t n, const float *x, float *y)
{
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        float x3 = v * v * v;
        float inner = 0.7978845608f * (v + 0.044715f * x3);
        y[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* shaders/norm/layer_norm_f64.wgsl:20-50 in double: per row, sequential
 * mean, two-pass biased variance, (x - mean) / sqrt(var + eps). */
BCO_API void bco_layer_norm_f64(long rows, long cols, double eps,
                                const float *x, double *y)
{
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        double *yr = y + r * cols;
        double sum = 0.0;
        for (long i = 0; i < cols; ++i) sum += (double)xr[i];
        double mean = sum / (double)cols;
        double var_sum = 0.0;
        for (long i = 0; i < cols; ++i) {
            double d = (double)xr[i] - mean;
            var_sum += d * d;
        }
        double sd = sqrt(var_sum / (double)cols + eps);
        for (long i = 0; i < cols; ++i) yr[i] = ((double)xr[i] - mean) / sd;
    }
}

/* layer_norm_f64.wgsl downcast to f32 (sqrt_f64 -> sqrt): the same steps
 * in f32 with sequential sums, one thread per row as the shader runs. */
BCO_API void bco_layer_norm_f32(long rows, long cols, float eps,
                                const float *x, float *y)
{
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        float sum = 0.0f;
        for (long i = 0; i < cols; ++i) sum = sum + xr[i];
        float mean = sum / (float)cols;
        float var_sum = 0.0f;
        for (long i = 0; i < cols; ++i) {
            float d = xr[i] - mean;
            var_sum = var_sum + d * d;
        }
        float variance = var_sum / (float)cols;
        float sd = sqrtf(variance + eps);
        for (long i = 0; i < cols; ++i) yr[i] = (xr[i] - mean) / sd;
    }
}

/* ------------------------------------------------------------------------
 * 5. Inline-data f64 handlers of the IPC wire paths (paths relative to
 *    crates/barracuda-core/src/ipc/methods/ of the reference)
 * ---------------------------------------------------------------------- */

/* The row softmax of ml.attention (ml/forward.rs:130-140) on one row:
 * max_val folded from -inf with f64::max (fmax: NaN entries skipped),
 * val = exp(val - max_val) with the sum accumulated in order, then each
 * value divided by the sum. */
static void ml_softmax_row(long cols, double *row)
{
    double mx = -INFINITY;
    for (long j = 0; j < cols; ++j) mx = fmax(mx, row[j]);
    double sum = 0.0;
    for (long j = 0; j < cols; ++j) {
        row[j] = exp(row[j] - mx);
        sum += row[j];
    }
    for (long j = 0; j < cols; ++j) row[j] /= sum;
}

BCO_API void bco_ml_softmax_rows_f64(long rows, long cols, const double *x,
                                     double *y)
{
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; ++r) {
        double *yr = y + r * cols;
        if (yr != x + r * cols) memcpy(yr, x + r * cols, (size_t)cols * sizeof(double));
        ml_softmax_row(cols, yr);
    }
}

/* ml.attention (ml/forward.rs:121-150) on row-major q [sq][dk], k [sk][dk],
 * v [sk][dv] into out [sq][dv]:
 *   scale = 1 / sqrt(dk)
 *   score[i][j] = (sum over d, in order, of q[i][d] * k[j][d]) * scale
 *                 (products rounded, then added: no fused multiply-add)
 *   the row softmax above
 *   out[i][c] = fma(w_ij, v[j][c], out[i][c]) over j in order, from 0. */
BCO_API void bco_ml_attention_f64(int sq, int sk, int dk, int dv,
                                  const double *q, const double *k,
                                  const double *v, double *out)
{
    const double scale = 1.0 / sqrt((double)dk);
    #pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < sq; ++i) {
        double *w = (double *)malloc((size_t)(sk > 0 ? sk : 1) * sizeof(double));
        const double *qi = q + (long)i * dk;
        for (int j = 0; j < sk; ++j) {
            const double *kj = k + (long)j * dk;
            double s = 0.0;
            for (int d = 0; d < dk; ++d) s += qi[d] * kj[d];
            w[j] = s * scale;
        }
        ml_softmax_row(sk, w);
        double *oi = out + (long)i * dv;
        for (int c = 0; c < dv; ++c) oi[c] = 0.0;
        for (int j = 0; j < sk; ++j) {
            const double *vj = v + (long)j * dv;
            for (int c = 0; c < dv; ++c) oi[c] = fma(w[j], vj[c], oi[c]);
        }
        free(w);
    }
}

/* tensor.matmul_inline (tensor.rs:540-548): lhs [m][k] times rhs [k][n],
 * sum = fma(lhs[i][p], rhs[p][j], sum) over p in order, from 0. */
BCO_API void bco_matmul_inline_f64(int m, int k, int n, const double *lhs,
                                   const double *rhs, double *out)
{
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            double sum = 0.0;
            for (int p = 0; p < k; ++p)
                sum = fma(lhs[(long)i * k + p], rhs[(long)p * n + j], sum);
            out[(long)i * n + j] = sum;
        }
}
