"""f64 GEMM on the MI355X FP64 matrix cores (bch_dgemm, GemmF64,
GemmCachedF64) vs the oracle.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-12 against a longdouble
product (oracle.gemm_longdouble); the reference's own algorithm restated in
f64 (oracle.gemm_f64_wgsl) is held to the same bar.  The reference tests'
vectors and integer-valued inputs are bit-exact.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import F64Buffer, GemmCachedF64, GemmF64
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-12


def _say(msg):
    print(msg, flush=True)


def _rel(x, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(x) - ref) / np.maximum(np.abs(ref), 1.0)))


def test_reference_vectors(dev):
    _say("dgemm reference vectors")
    assert GemmF64.execute(dev, [1, 2, 3, 4], [5, 6, 7, 8], 2, 2, 2, 1).tolist() == [19, 22, 43, 50]
    assert GemmF64.execute_gemm_ex(dev, [1, 3, 2, 4], [5, 6, 7, 8], 2, 2, 2, 1, 1.0, 0.0, True, False).tolist() == \
        [19, 22, 43, 50]
    assert GemmF64.execute_gemm_ex(dev, [1, 2, 3, 4], [5, 7, 6, 8], 2, 2, 2, 1, 1.0, 0.0, False, True).tolist() == \
        [19, 22, 43, 50]
    b9 = list(range(1, 10))
    got = GemmF64.execute(dev, [1, 0, 0, 0, 1, 0, 0, 0, 1, 2, 0, 0, 0, 2, 0, 0, 0, 2], b9 + b9, 3, 3, 3, 2)
    assert got.tolist() == b9 + [2 * x for x in b9]


@pytest.mark.parametrize("batch,m,k,n", [(1, 128, 128, 128), (1, 256, 512, 384), (1, 100, 33, 77), (1, 1, 1, 1),
                                         (1, 3, 17, 129), (4, 64, 80, 96), (2, 256, 64, 128)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_dgemm_vs_longdouble(dev, batch, m, k, n, ta, tb):
    _say(f"dgemm batch={batch} m={m} k={k} n={n} ta={ta} tb={tb}")
    rng = O.Lcg(batch + m * 3 + k * 5 + n * 7 + 2 * ta + tb)
    a = rng.uniform((batch * m * k,)).astype(np.float64) + rng.uniform((batch * m * k,)).astype(np.float64) * 1e-7
    b = rng.uniform((batch * k * n,)).astype(np.float64) + rng.uniform((batch * k * n,)).astype(np.float64) * 1e-7
    got = GemmF64.execute_gemm_ex(dev, a, b, m, k, n, batch, 1.0, 0.0, ta, tb)
    assert _rel(got, O.gemm_longdouble(a, b, m, k, n, batch, ta, tb)) <= TOL
    assert _rel(got, O.gemm_f64_wgsl(a, b, m, k, n, batch, trans_a=ta, trans_b=tb)) <= TOL


def test_dgemm_exact_on_integers(dev):
    _say("dgemm integers")
    rng = np.random.default_rng(4)
    for (m, k, n) in ((128, 256, 128), (50, 70, 90)):
        a = rng.integers(-64, 65, m * k).astype(np.float64)
        b = rng.integers(-64, 65, k * n).astype(np.float64)
        want = (a.astype(np.int64).reshape(m, k) @ b.astype(np.int64).reshape(k, n)).reshape(-1)
        assert np.array_equal(GemmF64.execute(dev, a, b, m, k, n, 1), want.astype(np.float64))


def test_alpha_beta_reads_c_only_when_beta_nonzero(dev):
    _say("dgemm alpha/beta")
    m = k = n = 128
    rng = O.Lcg(77)
    a = rng.uniform((m * k,)).astype(np.float64)
    b = rng.uniform((k * n,)).astype(np.float64)
    cin = rng.uniform((m * n,)).astype(np.float64)
    lib = dev._lib
    for alpha, beta, c0 in ((0.5, -2.0, cin), (3.0, 0.0, np.full(m * n, np.nan))):
        da, db = F64Buffer(dev, a.size).upload(a), F64Buffer(dev, b.size).upload(b)
        dc = F64Buffer(dev, m * n).upload(c0)
        with dev._lock:
            dev.check(lib.bch_dgemm(dev.ctx, 0, 0, 1, m, n, k, alpha, C.c_void_p(da.ptr), k, m * k,
                                    C.c_void_p(db.ptr), n, k * n, beta, C.c_void_p(dc.ptr), n, m * n), "dgemm")
        want = O.gemm_f64_wgsl(a, b, m, k, n, 1, alpha=alpha, beta=beta, c_in=c0)
        assert _rel(dc.to_vec(), want) <= TOL


def test_gemm_cached_non_square(dev):
    """GemmCachedF64 with m != n: every output element is computed."""
    _say("GemmCachedF64 m=40 k=64 n=200 batch=2")
    rng = O.Lcg(5)
    k, n, batch, m = 64, 200, 2, 40
    b = rng.uniform((batch * k * n,)).astype(np.float64)
    g = GemmCachedF64.new(dev, b, k, n, batch)
    for mm in (m, 7):
        a = rng.uniform((batch * mm * k,)).astype(np.float64)
        assert _rel(g.multiply(a, mm), O.gemm_longdouble(a, b, mm, k, n, batch)) <= TOL


def test_dgemm_2048_sampled_rows(dev):
    """A full-tile size with every CU busy; rows sampled against longdouble."""
    _say("dgemm 2048^3 sampled rows")
    n = 2048
    rng = O.Lcg(2)
    a = rng.uniform((n * n,)).astype(np.float64)
    b = rng.uniform((n * n,)).astype(np.float64)
    got = GemmF64.execute(dev, a, b, n, n, n, 1).reshape(n, n)
    B = b.astype(np.longdouble).reshape(n, n)
    for r in (0, 1, 777, 2047):
        ref = (a[r * n:(r + 1) * n].astype(np.longdouble) @ B).astype(np.float64)
        assert _rel(got[r], ref) <= TOL


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_dgemm_empty_k_batched(dev, ta, tb):
    """k == 0 with batch > 1: op(A) op(B) is the zero matrix, so C = 0
    (the reference's fresh C buffer scaled by beta); no shape error."""
    _say(f"dgemm batch=3 m=4 k=0 n=5 ta={ta} tb={tb}")
    got = GemmF64.execute_gemm_ex(dev, [], [], 4, 0, 5, 3, 1.0, 0.5, ta, tb)
    assert got.shape == (60,) and not np.any(got)


@pytest.mark.parametrize("batch,m,k,n", [(1, 2048, 2048, 128), (1, 128, 4096, 64), (3, 100, 1000, 37),
                                         (1, 64, 8192, 64), (2, 256, 2064, 256), (1, 1, 5000, 1)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)])
def test_dgemm_split_k_vs_longdouble(dev, batch, m, k, n, ta, tb):
    """Outputs with fewer 128 x 128 tiles than CUs and long k: the k range is
    split, the partials added in split order by a second kernel."""
    _say(f"dgemm split-k batch={batch} m={m} k={k} n={n} ta={ta} tb={tb}")
    rng = O.Lcg(batch * 11 + m + 3 * k + 7 * n + ta)
    a = rng.uniform((batch * m * k,)).astype(np.float64)
    b = rng.uniform((batch * k * n,)).astype(np.float64)
    got = GemmF64.execute_gemm_ex(dev, a, b, m, k, n, batch, 1.0, 0.0, ta, tb)
    assert _rel(got, O.gemm_longdouble(a, b, m, k, n, batch, ta, tb)) <= TOL
    again = GemmF64.execute_gemm_ex(dev, a, b, m, k, n, batch, 1.0, 0.0, ta, tb)
    assert np.array_equal(got, again)  # fixed summation order


def test_dgemm_split_k_alpha_beta_and_integers(dev):
    _say("dgemm split-k alpha/beta and integers")
    m, k, n = 128, 4096, 128
    rng = np.random.default_rng(8)
    a = rng.integers(-32, 33, m * k).astype(np.float64)
    b = rng.integers(-32, 33, k * n).astype(np.float64)
    want = (a.astype(np.int64).reshape(m, k) @ b.astype(np.int64).reshape(k, n)).reshape(-1)
    assert np.array_equal(GemmF64.execute(dev, a, b, m, k, n, 1), want.astype(np.float64))
    cin = rng.uniform(-1, 1, m * n)
    lib = dev._lib
    for alpha, beta, c0 in ((0.5, -2.0, cin), (3.0, 0.0, np.full(m * n, np.nan))):
        da, db = F64Buffer(dev, a.size).upload(a), F64Buffer(dev, b.size).upload(b)
        dc = F64Buffer(dev, m * n).upload(c0)
        with dev._lock:
            dev.check(lib.bch_dgemm(dev.ctx, 0, 0, 1, m, n, k, alpha, C.c_void_p(da.ptr), k, m * k,
                                    C.c_void_p(db.ptr), n, k * n, beta, C.c_void_p(dc.ptr), n, m * n), "dgemm")
        ref = alpha * want.astype(np.float64) + (beta * c0 if beta != 0.0 else 0.0)
        assert _rel(dc.to_vec(), ref) <= TOL


def _dgemm_raw(dev, ta, tb, batch, m, n, k, A, lda, sA, B, ldb, sB, ldc, sC, a_shift=0, b_shift=0):
    """bch_dgemm on host arrays laid out with the given leading dimensions and
    batch strides; a_shift / b_shift move the operand base by that many
    doubles (8 bytes each: not 16-byte aligned when odd)."""
    da = F64Buffer(dev, A.size + a_shift).upload(np.concatenate([np.zeros(a_shift), A]))
    db = F64Buffer(dev, B.size + b_shift).upload(np.concatenate([np.zeros(b_shift), B]))
    dc = F64Buffer(dev, batch * sC).upload(np.full(batch * sC, 7.25))
    with dev._lock:
        dev.check(dev._lib.bch_dgemm(dev.ctx, int(ta), int(tb), batch, m, n, k, 1.0,
                                     C.c_void_p(da.ptr + 8 * a_shift), lda, sA, C.c_void_p(db.ptr + 8 * b_shift),
                                     ldb, sB, 0.0, C.c_void_p(dc.ptr), ldc, sC), "dgemm")
    return dc.to_vec()


# Ragged shapes whose paired dimension is even take the 128-bit pair-guarded
# loads (every transpose; batched; split k); the odd and misaligned ones take
# the scalar guards.  Each result is compared with longdouble, the padding
# of C (ldc > n) must keep its fill.
@pytest.mark.parametrize("batch,m,k,n", [(1, 130, 34, 258), (3, 62, 98, 200), (1, 258, 2050, 130),
                                         (2, 100, 1000, 38), (1, 4, 4096, 6)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("pad,shift", [(0, 0), (2, 0), (2, 1)])
def test_dgemm_guarded_pair_loads(dev, batch, m, k, n, ta, tb, pad, shift):
    _say(f"dgemm guarded batch={batch} m={m} k={k} n={n} ta={ta} tb={tb} pad={pad} shift={shift}")
    rng = np.random.default_rng(batch * 7 + m + 3 * k + 5 * n + 2 * ta + tb + 11 * pad + shift)
    a = rng.uniform(-1, 1, (batch, k, m) if ta else (batch, m, k))
    b = rng.uniform(-1, 1, (batch, n, k) if tb else (batch, k, n))
    lda, ldb, ldc = a.shape[2] + pad, b.shape[2] + 2 * pad, n + pad
    sA, sB, sC = a.shape[1] * lda + pad, b.shape[1] * ldb, m * ldc + 2 * pad
    A = np.full(batch * sA, np.nan)  # padding reads would poison the sums
    B = np.full(batch * sB, np.nan)
    for z in range(batch):
        A[z * sA:z * sA + a.shape[1] * lda].reshape(a.shape[1], lda)[:, :a.shape[2]] = a[z]
        B[z * sB:z * sB + b.shape[1] * ldb].reshape(b.shape[1], ldb)[:, :b.shape[2]] = b[z]
    got = _dgemm_raw(dev, ta, tb, batch, m, n, k, A, lda, sA, B, ldb, sB, ldc, sC, a_shift=shift, b_shift=shift)
    want = O.gemm_longdouble(a.reshape(-1), b.reshape(-1), m, k, n, batch, ta, tb).reshape(batch, m, n)
    for z in range(batch):
        block = got[z * sC:z * sC + m * ldc].reshape(m, ldc)
        assert _rel(block[:, :n], want[z]) <= TOL
        assert np.all(block[:, n:] == 7.25)
        assert np.all(got[z * sC + m * ldc:(z + 1) * sC] == 7.25)
