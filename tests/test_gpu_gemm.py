"""f32 GEMM on the MI355X vs the oracle (bch_sgemm, bch_sgemm_strided_batched).

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle
(tolerances/mod.rs:44-54 scale).  The literal reference vectors are checked
at the reference tests' own tolerances.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import Tensor
from oracle import bc_oracle as O
from tests.conftest import case_inputs

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _mm(dev, a, b):
    ta = Tensor.from_data(a, list(a.shape), dev)
    tb = Tensor.from_data(b, list(b.shape), dev)
    return ta.matmul(tb).to_numpy()


def test_golden_vectors(dev, golden):
    for case in golden["matmul"]:
        _say(f"matmul golden {case['name']}")
        a, b = case_inputs(case)
        got = _mm(dev, a, b).reshape(-1)
        want = np.array(case["expected"])
        if case["tol"] == 0.0:
            assert np.array_equal(got, want.astype(np.float32)), case["name"]
        else:
            # the reference tests' absolute bound, widened to 1e-6 relative where
            # |C| is so large (6875 in the ramps) that it is below 2 ulp of f32
            bound = np.maximum(case["tol"], 1e-6 * np.abs(want))
            assert np.all(np.abs(got - want) <= bound), case["name"]
    for case in golden["batch_matmul"]:
        a = np.array(case["a"], dtype=np.float32).reshape(case["a_shape"])
        b = np.array(case["b"], dtype=np.float32).reshape(case["b_shape"])
        ta, tb = Tensor.from_data(a, case["a_shape"], dev), Tensor.from_data(b, case["b_shape"], dev)
        got = ta.batch_matmul(tb)
        assert got.shape() == [2, 2, 2]
        assert np.array_equal(got.to_vec(), np.array(case["expected"], dtype=np.float32))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (2, 3, 1), (7, 5, 3), (33, 65, 17), (100, 70, 33),
                                   (128, 128, 32), (256, 128, 64), (129, 257, 100), (512, 384, 160),
                                   (40, 11008, 64), (300, 4, 4096), (64, 64, 0), (256, 256, 0), (2048, 8192, 0), (4095, 4096, 0)])
def test_shapes_vs_f64(dev, m, n, k):
    _say(f"sgemm m={m} n={n} k={k}")
    rng = O.Lcg(m * 7 + n * 13 + k)
    a = rng.uniform((m, k))
    b = rng.uniform((k, n))
    got = _mm(dev, a, b) if k > 0 else None
    if k == 0:
        ta, tb = Tensor.empty([m, 0], dev), Tensor.empty([0, n], dev)
        got = ta.matmul(tb).to_numpy()
        assert not got.any()
        return
    ref = O.matmul_f64(a, b)
    assert O.max_rel_err(got, ref) <= TOL
    # integer-valued inputs: the MFMA path is exact
    ai = np.round(a * 8).astype(np.float32)
    bi = np.round(b * 8).astype(np.float32)
    exact = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32)
    assert np.array_equal(_mm(dev, ai, bi), exact)


@pytest.mark.parametrize("m", [1, 2, 8, 13, 32])
def test_skinny_decode_shapes(dev, m):
    """BASELINE config 4 shapes: M in {1, 8, 32}, K = 4096, N = 11008; X ~ N(0,1),
    W ~ N(0, 0.02), seed 3 (plus M = 2, 13 for the routing edges)."""
    _say(f"skinny m={m} k=4096 n=11008 seed 3")
    rng = O.Lcg(3)
    x = rng.normal((m, 4096))
    w = rng.normal((4096, 11008), 0.0, 0.02)
    got = _mm(dev, x, w)
    ref = O.matmul_f64(x, w)
    err = O.max_rel_err(got, ref)
    _say(f"  max rel err = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("m,n,k", [(1, 4, 1), (3, 12, 37), (4, 260, 1000), (5, 8, 3), (9, 1028, 333),
                                   (16, 4096, 4100), (17, 300, 77), (31, 1024, 5000), (32, 11008, 129)])
def test_skinny_ragged(dev, m, n, k):
    _say(f"skinny ragged m={m} n={n} k={k}")
    rng = O.Lcg(m * 100 + n + k)
    a = rng.normal((m, k))
    b = rng.normal((k, n), 0.0, 0.02)
    assert O.max_rel_err(_mm(dev, a, b), O.matmul_f64(a, b)) <= TOL


@pytest.mark.parametrize("m", [5, 8, 16, 17, 32, 48, 64])
def test_skinny_exact_integers(dev, m):
    """Small-integer inputs make every partial sum exact in f32, so the split-k
    stream-K path must match the int64 product bit for bit (K 4096, N 11008)."""
    _say(f"skinny exact integers m={m}")
    rng = O.Lcg(m + 7)
    a = np.round(rng.uniform((m, 4096)) * 3).astype(np.float32)
    b = np.round(rng.uniform((4096, 11008)) * 7).astype(np.float32)
    exact = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(_mm(dev, a, b), exact)


def test_skinny_long_k_more_workgroups_than_cus(dev):
    """K = 400000: a workgroup's A^T run would overflow LDS at one workgroup
    per CU, so the plan uses more workgroups (several rounds)."""
    m, n, k = 32, 256, 400000
    _say(f"skinny long k m={m} n={n} k={k}")
    rng = O.Lcg(4)
    a = rng.normal((m, k))
    b = rng.normal((k, n), 0.0, 0.02)
    assert O.max_rel_err(_mm(dev, a, b), O.matmul_f64(a, b)) <= TOL


@pytest.mark.parametrize("m,n,k,lda_pad,a_off", [
    (20, 4, 4, 0, 0),        # one 32-row unit, K < 32 (tail rows zeroed)
    (24, 100, 36, 0, 0),     # ragged last column group, K % 32 != 0
    (32, 8, 4096, 0, 0),     # fewer units than CUs
    (17, 520, 68, 4, 0),     # lda = k + 4 (still a multiple of 4)
    (32, 512, 640, 1, 0),    # lda % 4 != 0: the 16x16x4 fallback
    (18, 256, 64, 0, 1),     # A misaligned by one float: the fallback
])
def test_skinny_m_over_16_routes(dev, m, n, k, lda_pad, a_off):
    """16 < m <= 32: the 32x32x2 kernel (aligned A, K % 4 == 0) and its
    fallbacks, called through the C ABI with an explicit lda."""
    _say(f"skinny m={m} n={n} k={k} lda=k+{lda_pad} a_off={a_off}")
    rng = O.Lcg(m + n + k)
    a = rng.normal((m, k))
    b = rng.normal((k, n), 0.0, 0.02)
    lda = k + lda_pad
    a_buf = np.zeros(a_off + m * lda, dtype=np.float32)
    a_buf[a_off:].reshape(m, lda)[:, :k] = a
    ta = Tensor.from_data(a_buf, [a_buf.size], dev)
    tb = Tensor.from_data(b, [k, n], dev)
    tc = Tensor.empty([m, n], dev)
    dev.check(dev._lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(ta.ptr + 4 * a_off), lda, C.c_void_p(tb.ptr), n,
                                 C.c_void_p(tc.ptr), n), "sgemm")
    assert O.max_rel_err(tc.to_numpy(), O.matmul_f64(a, b)) <= TOL


@pytest.mark.parametrize("m,n,k,lda_pad,a_off,skinny", [
    (33, 11008, 4096, 0, 0, True),   # the config's K and N, one row into the second block
    (48, 11008, 4096, 0, 0, True),
    (64, 11008, 4096, 0, 0, True),
    (40, 100, 36, 0, 0, True),       # ragged last column group, K % 32 != 0
    (64, 8, 4096, 0, 0, True),       # fewer units than CUs
    (50, 520, 68, 4, 0, True),       # lda = k + 4 (still a multiple of 4)
    (64, 512, 640, 1, 0, False),     # lda % 4 != 0: the tiles
    (45, 256, 64, 0, 1, False),      # A misaligned by one float: the tiles
])
def test_skinny_64_rows(dev, m, n, k, lda_pad, a_off, skinny):
    """32 < m <= 64: the 32x32x2 stream-K kernel with two 32-row blocks per streamed unit of B
    (aligned A, K % 4 == 0), else the tile path; called through the C ABI with an explicit lda."""
    if lda_pad == 0 and a_off == 0:
        name = dev._lib.bch_sgemm_kernel_name(m, n, k).decode()
        assert (name == "sgemm_skinny_w32<2>") == skinny, name
    _say(f"skinny 64-row m={m} n={n} k={k} lda=k+{lda_pad} a_off={a_off}")
    rng = O.Lcg(m * 3 + n + k)
    a = rng.normal((m, k))
    b = rng.normal((k, n), 0.0, 0.02)
    lda = k + lda_pad
    a_buf = np.zeros(a_off + m * lda, dtype=np.float32)
    a_buf[a_off:].reshape(m, lda)[:, :k] = a
    ta = Tensor.from_data(a_buf, [a_buf.size], dev)
    tb = Tensor.from_data(b, [k, n], dev)
    tc = Tensor.empty([m, n], dev)
    call = lambda: dev._lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(ta.ptr + 4 * a_off), lda, C.c_void_p(tb.ptr), n,
                                      C.c_void_p(tc.ptr), n)
    dev.check(call(), "sgemm")
    got = tc.to_numpy()
    assert O.max_rel_err(got, O.matmul_f64(a, b)) <= TOL
    dev.check(call(), "sgemm")
    assert np.array_equal(tc.to_numpy(), got), "not deterministic"


def test_skinny_repeated_calls_and_unaligned_a(dev):
    _say("skinny repeated calls / unaligned A")
    rng = O.Lcg(99)
    a = rng.normal((9, 640))
    b = rng.normal((640, 512))
    ref = O.matmul_f64(a, b)
    tb = Tensor.from_data(b, [640, 512], dev)
    ta = Tensor.from_data(np.concatenate([[0.0], a.reshape(-1)]).astype(np.float32), [1 + a.size], dev)
    for _ in range(3):  # workspace reuse across calls of different shapes
        tc = Tensor.empty([9, 512], dev)
        dev.check(dev._lib.bch_sgemm(dev.ctx, 9, 512, 640, C.c_void_p(ta.ptr + 4), 640, C.c_void_p(tb.ptr), 512,
                                     C.c_void_p(tc.ptr), 512), "sgemm")
        assert O.max_rel_err(tc.to_numpy(), ref) <= TOL
        small = _mm(dev, a[:2, :100].copy(), b[:100, :8].copy())
        assert O.max_rel_err(small, O.matmul_f64(a[:2, :100].copy(), b[:100, :8].copy())) <= TOL


def test_leading_dimensions_and_unaligned(dev):
    _say("sgemm with lda/ldb/ldc > natural and an odd offset")
    m, n, k = 96, 160, 72
    rng = O.Lcg(77)
    A = rng.uniform((m, k + 5))
    B = rng.uniform((k, n + 3))
    ta = Tensor.from_data(A, [m, k + 5], dev)
    tb = Tensor.from_data(B, [k, n + 3], dev)
    tc = Tensor.empty([m, n + 7], dev)
    dev.check(dev._lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(ta.ptr), k + 5, C.c_void_p(tb.ptr), n + 3,
                                 C.c_void_p(tc.ptr), n + 7), "sgemm")
    got = tc.to_numpy()[:, :n]
    ref = O.matmul_f64(np.ascontiguousarray(A[:, :k]), np.ascontiguousarray(B[:, :n]))
    assert O.max_rel_err(got, ref) <= TOL
    # A starting 4 bytes into an allocation (not 16-byte aligned)
    ta2 = Tensor.from_data(np.concatenate([[0.0], A.reshape(-1)]).astype(np.float32), [1 + A.size], dev)
    tc2 = Tensor.empty([m, n], dev)
    dev.check(dev._lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(ta2.ptr + 4), k + 5, C.c_void_p(tb.ptr),
                                 n + 3, C.c_void_p(tc2.ptr), n), "sgemm")
    assert O.max_rel_err(tc2.to_numpy(), ref) <= TOL


LARGE_TILE_CASES = [  # (m, n, k, the kernel the shape takes)
    (4096, 4096, 256, "sgemm_mfma_kernel<256,256,32,false>"),
    (4096, 3968, 64, "sgemm_mfma_kernel<256,256,32,true,v4>"),
    (4095, 4096, 33, "sgemm_mfma_kernel<256,256,32,true>"),
    (8192, 1024, 64, "sgemm_mfma_kernel<256,128,32,false>"),
    (8192, 1020, 68, "sgemm_mfma_kernel<256,128,32,true,v4>"),
    (8190, 1024, 62, "sgemm_mfma_kernel<256,128,32,true>"),
    (2048, 2048, 512, "sgemm_mfma_kernel<128,128,32,false>"),
    (4100, 4096, 300, "sgemm_mfma_kernel<128,128,32,true,v4>"),
    (2000, 2000, 95, "sgemm_mfma_kernel<128,128,32,true>"),
]


@pytest.mark.parametrize("m,n,k,kernel", LARGE_TILE_CASES)
def test_large_tile_paths(dev, m, n, k, kernel):
    """Every block tile (256x256, 256x128, 128x128) with every load mode: unguarded (whole tiles,
    aligned), guarded float4 loads (ragged M or N, K and N multiples of 4) and guarded scalar
    loads (K or N not a multiple of 4).  Sampled rows and columns vs f64, rows and columns on
    both sides of tile boundaries and the ragged edges."""
    assert dev._lib.bch_sgemm_kernel_name(m, n, k).decode() == kernel
    _say(f"sgemm large tiles m={m} n={n} k={k} ({kernel})")
    rng = O.Lcg(m + n + k)
    a = rng.uniform((m, k))
    b = rng.uniform((k, n))
    got = _mm(dev, a, b)
    rows = [0, 1, 127, 128, 255, 256, m // 2, m - 2, m - 1]
    assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL
    cols = [0, 127, 128, 255, 256, n - 3, n - 1]
    assert O.max_rel_err(got[:, cols], a.astype(np.float64) @ b[:, cols].astype(np.float64)) <= TOL


# the last three take several rounds of slices over 86 / 172 / 86 tiles
SPLIT_K_CASES = [(1024, 1024, 4096), (512, 512, 8192), (300, 4, 4096), (96, 4096, 4096), (200, 1000, 2048),
                 (128, 11008, 4096), (192, 11008, 4096), (96, 11008, 4096)]


@pytest.mark.parametrize("m,n,k", SPLIT_K_CASES)
def test_split_k_vs_f64(dev, m, n, k):
    """Tiles filling less than one round: K is cut into slices of whole k-tiles, the slices run
    as one batched launch (one or several rounds) into the workspace and sgemm_splitk_reduce
    adds them in slice order.  Aligned and ragged (m 300, 192, 96, n 4 and 1000: the
    float4-guarded tiles), full f64 comparison on sampled rows and every column; repeated
    calls are bit-identical."""
    name = dev._lib.bch_sgemm_kernel_name(m, n, k).decode()
    assert name.endswith("+sgemm_splitk_reduce"), name
    _say(f"sgemm split-k m={m} n={n} k={k} ({name})")
    rng = O.Lcg(m * 3 + n + k)
    a = rng.uniform((m, k))
    b = rng.uniform((k, n))
    got = _mm(dev, a, b)
    rows = sorted(set(r for r in (0, 1, 63, 64, 127, m // 2, m - 1) if r < m))
    assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL
    assert np.array_equal(got, _mm(dev, a, b)), "not deterministic"


def test_split_k_exact_on_integers(dev):
    """Small integers: every partial sum is exact in f32, whatever the slice order."""
    rng = np.random.default_rng(17)
    for m, n, k in ((1024, 1024, 4096), (64, 4096, 4096)):
        _say(f"sgemm split-k integers m={m} n={n} k={k}")
        a = rng.integers(-8, 9, (m, k)).astype(np.float32)
        b = rng.integers(-8, 9, (k, n)).astype(np.float32)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        assert np.array_equal(_mm(dev, a, b), want), (m, n, k)


# 64 x 64 x 64 tiles: shapes whose usual tiles fill less than one round and whose k is short
SMALL_CASES = [(128, 128, 128), (256, 256, 256), (192, 320, 256), (128, 1024, 512), (512, 512, 512), (768, 768, 768),
               (1024, 1024, 1024), (1024, 2048, 1024)]


@pytest.mark.parametrize("m,n,k", SMALL_CASES)
def test_small_tiles_vs_f64(dev, m, n, k):
    """The 64 x 64 x 64 tile (one 32 x 32 MFMA block per wavefront, no k split): every element
    against f64 (inputs scaled by 1/sqrt(k)), then the same shape with the operands' leading
    dimensions padded by 4 (the same kernel) and with A one float off 16-byte alignment (the
    usual tiles), and the linear layer's forms ([n][k] weights, bias, ReLU and GELU)."""
    name = dev._lib.bch_sgemm_kernel_name(m, n, k).decode()
    assert name == "sgemm_mfma_kernel<64,64,64,false>", name
    _say(f"sgemm small tiles m={m} n={n} k={k}")
    rng = O.Lcg(m * 5 + n * 3 + k)
    a = rng.uniform((m, k)) / np.float32(np.sqrt(k))
    b = rng.uniform((k, n))
    want = a.astype(np.float64) @ b.astype(np.float64)
    got = _mm(dev, a, b)
    assert O.max_rel_err(got, want) <= TOL
    assert np.array_equal(got, _mm(dev, a, b)), "not deterministic"
    lib = dev._lib
    for pad, shift in ((4, 0), (0, 1)):
        ap = np.zeros(m * (k + pad) + shift, dtype=np.float32)
        ap[shift:].reshape(m, k + pad)[:, :k] = a
        bp = np.zeros((k, n + pad), dtype=np.float32)
        bp[:, :n] = b
        ta, tb = Tensor.from_data(ap, [ap.size], dev), Tensor.from_data(bp, [k, n + pad], dev)
        tc = Tensor.empty([m, n], dev)
        with dev._lock:
            dev.check(lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(ta.ptr + 4 * shift), k + pad, C.c_void_p(tb.ptr),
                                    n + pad, C.c_void_p(tc.ptr), n), "sgemm")
        assert O.max_rel_err(tc.to_numpy(), want) <= TOL, (pad, shift)
    w = rng.uniform((n, k))
    bias = rng.uniform((n,))
    tx, tw, tbias = (Tensor.from_data(x, list(x.shape), dev) for x in (a, w, bias))
    lin = a.astype(np.float64) @ w.astype(np.float64).T + bias.astype(np.float64)
    for act in (1, 2):  # BCH_ACT_RELU, BCH_ACT_GELU
        ty = Tensor.empty([m, n], dev)
        with dev._lock:
            dev.check(lib.bch_sgemm_ex(dev.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr), k,
                                       C.c_void_p(tbias.ptr), act, C.c_void_p(ty.ptr), n), "sgemm_ex")
        ref = np.maximum(lin, 0.0) if act == 1 else O.gelu_f64(lin.astype(np.float32))
        assert O.max_rel_err(ty.to_numpy(), ref) <= TOL, act


def test_small_tiles_exact_on_integers_and_batched(dev):
    """Small integers are exact in f32 whatever the order; batches of small shapes take the
    same tiles (grid.y = batch)."""
    rng = np.random.default_rng(23)
    a = rng.integers(-8, 9, (512, 1024)).astype(np.float32)
    b = rng.integers(-8, 9, (1024, 768)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(_mm(dev, a, b), want)
    _say("batched small tiles 3x(192x320x256)")
    r = O.Lcg(31)
    ab, bb = r.uniform((3, 192, 256)), r.uniform((3, 256, 320))
    ta, tb = Tensor.from_data(ab, [3, 192, 256], dev), Tensor.from_data(bb, [3, 256, 320], dev)
    got = ta.batch_matmul(tb).to_numpy()
    for i in range(3):
        assert O.max_rel_err(got[i], ab[i].astype(np.float64) @ bb[i].astype(np.float64)) <= TOL, i


HYBRID_CASES = [(3072, 3072, 1024, "sgemm_mfma_kernel<128,128,32,false,hyb>+sgemm_tail_reduce"),
                (3000, 3000, 1024, "sgemm_mfma_kernel<128,128,32,true,v4,hyb>+sgemm_tail_reduce"),
                (5120, 5120, 1024, "sgemm_mfma_kernel<256,128,32,false,hyb>+sgemm_tail_reduce"),
                (4100, 4100, 1024, "sgemm_mfma_kernel<256,128,32,true,v4,hyb>+sgemm_tail_reduce"),
                (6144, 6144, 1536, "sgemm_mfma_kernel<256,256,32,false,hyb>+sgemm_tail_reduce"),
                (6000, 6000, 3200, "sgemm_mfma_kernel<256,256,32,true,v4,hyb>+sgemm_tail_reduce")]


@pytest.mark.parametrize("m,n,k,kernel", HYBRID_CASES)
def test_hybrid_vs_f64(dev, m, n, k, kernel):
    """Tiles leaving the last round part-filled: whole rounds of tiles, then the leftover tiles
    in k-slices whose sums sgemm_tail_reduce adds in slice order.  Every tile size with
    unguarded and float4-guarded loads; rows across every tile row and columns across every
    tile column (so every whole and every split tile is compared with f64); repeated calls
    are bit-identical."""
    assert dev._lib.bch_sgemm_kernel_name(m, n, k).decode() == kernel
    _say(f"sgemm hybrid m={m} n={n} k={k} ({kernel})")
    rng = O.Lcg(m + 5 * n + 3 * k)
    a = rng.uniform((m, k))
    b = rng.uniform((k, n))
    got = _mm(dev, a, b)
    rows = sorted(r for r in {0, 1, m - 1} | {t * 128 + (t * 37) % 128 for t in range((m + 127) // 128)} if r < m)
    assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL
    cols = sorted(c for c in {0, n - 1} | {t * 128 + (t * 53) % 128 for t in range((n + 127) // 128)} if c < n)
    assert O.max_rel_err(got[:, cols], a.astype(np.float64) @ b[:, cols].astype(np.float64)) <= TOL
    assert np.array_equal(got, _mm(dev, a, b)), "not deterministic"


def test_hybrid_exact_on_integers(dev):
    """Small integers: every slice's sums are exact in f32, so the split tiles equal the
    whole-tile products bit for bit."""
    rng = np.random.default_rng(31)
    for m, n, k in ((3072, 3072, 1024), (4100, 4100, 1024)):
        _say(f"sgemm hybrid integers m={m} n={n} k={k}")
        a = rng.integers(-8, 9, (m, k)).astype(np.float32)
        b = rng.integers(-8, 9, (k, n)).astype(np.float32)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        assert np.array_equal(_mm(dev, a, b), want), (m, n, k)


MIXED_CASES = [(4096, 11008, 4096, "columns"), (11008, 4096, 4096, "rows"), (4096, 11000, 4096, "columns"),
               (11000, 4096, 4096, "rows"), (4100, 4096, 4096, "rows"), (2048, 11008, 4096, "columns")]


def _seam_sample(size: int):
    """One index in every 128 block, both ends, and both sides of the splits the mixed plan
    takes at these sizes (4096, 8192)."""
    idx = {0, size - 1, 4095, 4096, 8191, 8192} | {t * 128 + (t * 37) % 128 for t in range((size + 127) // 128)}
    return sorted(i for i in idx if i < size)


@pytest.mark.parametrize("m,n,k,axis", MIXED_CASES)
def test_mixed_vs_f64(dev, m, n, k, axis):
    """The mixed plan: whole rounds of 256x256 tiles on the first rows (columns) of C, then the
    rest planned on its own (data-parallel, split-K or hybrid; aligned and float4-guarded).
    Rows across every 128-row block and columns across every 128-column block, the seam
    between the two launches included, against f64 (B scaled by 1/sqrt(k)); repeated calls are
    bit-identical."""
    name = dev._lib.bch_sgemm_kernel_name(m, n, k).decode()
    assert f" {axis} then " in name, name
    _say(f"sgemm mixed m={m} n={n} k={k} ({name})")
    rng = O.Lcg(m + 7 * n + k)
    a = rng.uniform((m, k))
    # B scaled by 1/sqrt(k): outputs of order 1, so the bar measures the plan, not f32 rounding
    # of sums of order sqrt(k) (the exact-integer test below pins every element bit for bit)
    b = (rng.uniform((k, n)) / np.float32(np.sqrt(k))).astype(np.float32)
    got = _mm(dev, a, b)
    rows = _seam_sample(m)
    assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL
    cols = _seam_sample(n)
    assert O.max_rel_err(got[:, cols], a.astype(np.float64) @ b[:, cols].astype(np.float64)) <= TOL
    assert np.array_equal(got, _mm(dev, a, b)), "not deterministic"


def test_mixed_exact_on_integers(dev):
    """Small integers: every product is exact in f32 whatever the plan, so both launches of the
    mixed plan (and the split-K rest) match the integer product bit for bit."""
    rng = np.random.default_rng(41)
    for m, n, k in ((4096, 4100, 4096), (4100, 4096, 4096)):
        _say(f"sgemm mixed integers m={m} n={n} k={k}")
        a = rng.integers(-8, 9, (m, k)).astype(np.float32)
        b = rng.integers(-8, 9, (k, n)).astype(np.float32)
        # every partial sum is an integer below 2^18: the float64 product is exact
        want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
        assert np.array_equal(_mm(dev, a, b), want), (m, n, k)


def test_mixed_linear_bias_gelu(dev):
    """The linear layer (bch_sgemm_ex, [out, in] weights, bias, GELU) on the mixed plan: the
    rest's weights, bias and output start at column 8192 (weight row 8192)."""
    m, n, k = 4096, 11008, 4096
    _say(f"linear mixed m={m} n={n} k={k} bias + GELU")
    rng = O.Lcg(4242)
    x = rng.uniform((m, k))
    w = (rng.uniform((n, k)) / np.float32(np.sqrt(k))).astype(np.float32)
    bias = rng.uniform((n,))
    tx, tw, tb = (Tensor.from_data(t, list(t.shape), dev) for t in (x, w, bias))
    ty = Tensor.empty([m, n], dev)
    dev.check(dev._lib.bch_sgemm_ex(dev.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr), k,
                                    C.c_void_p(tb.ptr), 2, C.c_void_p(ty.ptr), n), "sgemm_ex")
    got = ty.to_numpy().reshape(m, n)
    rows = _seam_sample(m)[::3]
    pre = x[rows].astype(np.float64) @ w.T.astype(np.float64) + bias.astype(np.float64)
    assert O.max_rel_err(got[rows], O.gelu_f64(pre.astype(np.float32))) <= TOL
    cols = _seam_sample(n)
    pre = x.astype(np.float64) @ w[cols].T.astype(np.float64) + bias[cols].astype(np.float64)
    assert O.max_rel_err(np.ascontiguousarray(got[:, cols]), O.gelu_f64(pre.astype(np.float32))) <= TOL


def test_config_4096_cubed(dev):
    """BASELINE config 3a: 4096^3, U[-1,1), seed 2; f64 oracle on sampled rows."""
    _say("sgemm 4096^3 seed 2")
    rng = O.Lcg(2)
    a = rng.uniform((4096, 4096))
    b = rng.uniform((4096, 4096))
    got = _mm(dev, a, b)
    # one row in each of the 16 tile rows of 256 (the position inside the tile
    # moves with the tile) plus edge and interior rows: every 256x256 output
    # tile has a whole checked row
    rows = sorted({0, 1, 127, 128, 2047, 2048, 4095} | set(range(513, 4096, 257)) |
                  {t * 256 + (t * 37 + 11) % 256 for t in range(16)})
    ref = O.matmul_f64(a, b, rows=rows)
    err = O.max_rel_err(got[rows], ref)
    _say(f"  max rel err ({len(rows)} sampled rows) = {err:.3e}")
    assert err <= TOL
    # and one column in each of the 16 tile columns: C[:, j] = A @ B[:, j]
    cols = sorted({0, 31, 32, 4000, 4095} | {t * 256 + (t * 53 + 29) % 256 for t in range(16)})
    refc = a.astype(np.float64) @ b[:, cols].astype(np.float64)
    errc = O.max_rel_err(got[:, cols], refc)
    _say(f"  max rel err ({len(cols)} sampled columns) = {errc:.3e}")
    assert errc <= TOL
    assert {r // 256 for r in rows} == set(range(16)) and {c // 256 for c in cols} == set(range(16))


def test_config_batched_16x1024(dev):
    """BASELINE config 3b: batch 16 of 1024^3, U[-1,1), seed 2."""
    _say("batched sgemm 16x1024^3 seed 2")
    rng = O.Lcg(2)
    a = rng.uniform((16, 1024, 1024))
    b = rng.uniform((16, 1024, 1024))
    ta, tb = Tensor.from_data(a, [16, 1024, 1024], dev), Tensor.from_data(b, [16, 1024, 1024], dev)
    got = ta.batch_matmul(tb).to_numpy()
    # every batch, one row from each 256-row tile (the position inside the
    # tile moves with the batch) plus the first and last rows; and a column
    # from each 256-column tile
    for bi in range(16):
        rows = sorted({0, 1023} | {t * 256 + (bi * 37 + t * 101) % 256 for t in range(4)})
        ab, bb = np.ascontiguousarray(a[bi]), np.ascontiguousarray(b[bi])
        ref = O.matmul_f64(ab, bb, rows=rows)
        err = O.max_rel_err(got[bi][rows], ref)
        cols = [t * 256 + (bi * 53 + t * 29) % 256 for t in range(4)]
        errc = O.max_rel_err(got[bi][:, cols], ab.astype(np.float64) @ bb[:, cols].astype(np.float64))
        assert err <= TOL and errc <= TOL, (bi, rows, cols, err, errc)
    # batches are independent: the 16 batches in reverse order (the same kernel; fewer batches
    # split over k, which rounds differently) reproduce them bit for bit
    a2, b2 = np.ascontiguousarray(a[::-1]), np.ascontiguousarray(b[::-1])
    rev = Tensor.from_data(a2, [16, 1024, 1024], dev).batch_matmul(Tensor.from_data(b2, [16, 1024, 1024], dev))
    rev = rev.to_numpy()
    assert all(np.array_equal(rev[15 - i], got[i]) for i in range(16))
    single = _mm(dev, np.ascontiguousarray(a[3]), np.ascontiguousarray(b[3]))
    assert O.max_rel_err(single, got[3].astype(np.float64)) <= TOL


@pytest.mark.parametrize("batch,m,n,k", [(20, 1024, 1024, 256), (72, 512, 512, 64), (24, 1024, 768, 128),
                                         (8, 192, 320, 256)])
def test_batched_xcd_runs(dev, batch, m, n, k):
    """Batched launches whose (batch, tile) slots are handed to the XCDs in contiguous runs
    (2.5 batches a run at 20 x 16 tiles, 9 at 72 x 4, 24 x 12 tiles, and the 64 x 64 tiles at
    8 x 15): every tile of every batch against f64 (one row per 256-row tile and one column per
    256-column tile, at positions that move with the batch; every element below 256 rows), and
    the batches in reverse order reproduce them bit for bit."""
    _say(f"batched xcd runs {batch}x{m}x{n}x{k}")
    rng = O.Lcg(batch * 7 + m + n + k)
    a = rng.uniform((batch, m, k))
    b = rng.uniform((batch, k, n))
    ta, tb = Tensor.from_data(a, [batch, m, k], dev), Tensor.from_data(b, [batch, k, n], dev)
    got = ta.batch_matmul(tb).to_numpy()
    for bi in range(batch):
        rows = sorted({t * 256 + (bi * 37 + t * 101) % 256 for t in range(m // 256)} | {(bi * 13) % m})
        cols = sorted({t * 256 + (bi * 53 + t * 29) % 256 for t in range(n // 256)} | {(bi * 7) % n})
        if m < 256:
            rows = list(range(m))
        ab, bb = np.ascontiguousarray(a[bi]), np.ascontiguousarray(b[bi])
        err = O.max_rel_err(got[bi][rows], O.matmul_f64(ab, bb, rows=rows))
        errc = O.max_rel_err(got[bi][:, cols], ab.astype(np.float64) @ bb[:, cols].astype(np.float64))
        assert err <= TOL and errc <= TOL, (bi, err, errc)
    a2, b2 = np.ascontiguousarray(a[::-1]), np.ascontiguousarray(b[::-1])
    rev = Tensor.from_data(a2, [batch, m, k], dev).batch_matmul(Tensor.from_data(b2, [batch, k, n], dev)).to_numpy()
    assert all(np.array_equal(rev[batch - 1 - i], got[i]) for i in range(batch))


@pytest.mark.parametrize("batch,m,n,k", [(2, 1024, 1024, 2048), (4, 512, 512, 4096), (8, 256, 256, 8192),
                                         (3, 300, 200, 2048), (5, 130, 260, 1024)])
def test_batched_split_k(dev, batch, m, n, k):
    """Batches whose tiles together fill less than one round of the CUs split over k too
    (slices in grid.z, partials per batch and slice, a batch-aware reduce); aligned and ragged
    shapes, each batch against f64 on sampled rows and every column; repeated calls are
    bit-identical."""
    _say(f"batched split-k {batch}x{m}x{n}x{k}")
    rng = O.Lcg(batch * 1000 + m + n + k)
    a = rng.uniform((batch, m, k))
    b = rng.uniform((batch, k, n))
    ta, tb = Tensor.from_data(a, [batch, m, k], dev), Tensor.from_data(b, [batch, k, n], dev)
    got = ta.batch_matmul(tb).to_numpy()
    for bi in range(batch):
        rows = sorted({0, m - 1, m // 2, (bi * 37) % m})
        assert O.max_rel_err(got[bi][rows], O.matmul_f64(np.ascontiguousarray(a[bi]), np.ascontiguousarray(b[bi]),
                                                         rows=rows)) <= TOL, bi
    assert np.array_equal(ta.batch_matmul(tb).to_numpy(), got), "not deterministic"


def test_batched_ragged(dev):
    _say("batched sgemm ragged 3x(37x45x29)")
    rng = O.Lcg(5)
    a = rng.uniform((3, 37, 29))
    b = rng.uniform((3, 29, 45))
    ta, tb = Tensor.from_data(a, [3, 37, 29], dev), Tensor.from_data(b, [3, 29, 45], dev)
    got = ta.batch_matmul(tb).to_numpy()
    for i in range(3):
        assert O.max_rel_err(got[i], O.matmul_f64(np.ascontiguousarray(a[i]), np.ascontiguousarray(b[i]))) <= TOL
