"""The linear layer (bch_sgemm_ex: transposed weights, fused bias + ReLU)
and nn::fused_mlp on the MI355X vs the oracle.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle
(oracle.fused_mlp_f64 / numpy float64); the reference's own f32 algorithm
(linear_f64.wgsl + relu_f64.wgsl, oracle.linear_f32) is held to the same
bar on the same inputs.  Integer-valued inputs are bit-exact.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import Activation, Tensor, fused_mlp
from barracuda_amd import _native as N
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _up(dev, a):
    return Tensor.from_data(a, list(a.shape), dev)


def _sgemm_ex(dev, transb, x, w, bias, act):
    m, k = x.shape
    n = w.shape[0] if transb else w.shape[1]
    tx, tw = _up(dev, x), _up(dev, w)
    tb = _up(dev, bias) if bias is not None else None
    ty = Tensor.empty([m, n], dev)
    with dev._lock:
        dev.check(dev._lib.bch_sgemm_ex(dev.ctx, transb, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr),
                                        k if transb else n, C.c_void_p(tb.ptr) if tb else None, act,
                                        C.c_void_p(ty.ptr), n), "sgemm_ex")
    return ty.to_numpy()


def _ref(x, w, bias, transb, relu):
    y = x.astype(np.float64) @ (w.astype(np.float64).T if transb else w.astype(np.float64))
    if bias is not None:
        y = y + bias.astype(np.float64)
    return np.maximum(y, 0.0) if relu else y


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (512, 768, 1024), (100, 77, 33), (1, 1024, 512),
                                   (8, 11008, 256), (32, 512, 4096), (300, 129, 64), (500, 772, 1028),
                                   (260, 1000, 4), (64, 4096, 4096), (200, 1000, 2048), (3072, 1024, 3072),
                                   (3000, 3000, 1000), (3072, 3072, 512), (3000, 3000, 1024)])
@pytest.mark.parametrize("transb", [0, 1])
def test_sgemm_ex_vs_f64(dev, m, n, k, transb):
    _say(f"sgemm_ex m={m} n={n} k={k} transb={transb}")
    rng = O.Lcg(m + 3 * n + 7 * k + transb)
    x = rng.uniform((m, k))
    w = rng.uniform((n, k) if transb else (k, n))
    bias = rng.uniform((n,))
    for act, b in ((N.BCH_ACT_RELU, bias), (N.BCH_ACT_NONE, bias), (N.BCH_ACT_RELU, None), (N.BCH_ACT_NONE, None)):
        got = _sgemm_ex(dev, transb, x, w, b, act)
        assert O.max_rel_err(got, _ref(x, w, b, transb, act == N.BCH_ACT_RELU)) <= TOL, (act, b is None)


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (8, 4096, 4096), (32, 1024, 4096), (5, 300, 100), (17, 77, 36),
                                   (16, 129, 68), (32, 4, 4), (2, 200, 1028), (33, 11008, 4096), (64, 8200, 1000),
                                   (40, 9000, 4096)])
def test_sgemm_ex_transposed_decode_shapes(dev, m, n, k):
    """m <= 32 with [n][k] weights: the weight-row-streaming kernels, bias + ReLU in their epilogue;
    32 < m <= 64 at n >= 8192: the same kernels twice, on rows 0..31 and 32..m-1 (the second pass
    on the whole-row kernel for 33 and 40)."""
    _say(f"sgemm_ex transposed decode m={m} n={n} k={k}")
    rng = O.Lcg(m * 11 + n + k)
    x = rng.normal((m, k))
    w = rng.normal((n, k), 0.0, 0.05)
    bias = rng.normal((n,))
    for act, b in ((N.BCH_ACT_RELU, bias), (N.BCH_ACT_NONE, None)):
        got = _sgemm_ex(dev, 1, x, w, b, act)
        assert O.max_rel_err(got, _ref(x, w, b, True, act == N.BCH_ACT_RELU)) <= TOL, act


@pytest.mark.parametrize("m,n,k", [(8, 64, 16384), (32, 96, 8192), (13, 1000, 2100), (20, 11008, 4096),
                                   (6, 33, 260)])
def test_sgemm_ex_transposed_split_groups(dev, m, n, k):
    """The in-kernel split-k combine of the 4 < m <= 32 path: a 32-row group spread over many
    workgroups (n 64, k 16384: one unit per workgroup, 63 contributors per owner; n 96, k 8192),
    k not a multiple of 256 (2100, 260), the decode shape at m = 20, and a ragged last group
    (n 33).  Repeated calls reuse the workspace and its flags: each result is bit-identical."""
    _say(f"sgemm_ex transposed split groups m={m} n={n} k={k}")
    rng = O.Lcg(7 * m + n + k)
    x = rng.normal((m, k))
    w = rng.normal((n, k), 0.0, 0.05)
    bias = rng.normal((n,))
    for act, b in ((N.BCH_ACT_RELU, bias), (N.BCH_ACT_GELU, None)):
        first = _sgemm_ex(dev, 1, x, w, b, act)
        want = _ref(x, w, b, True, False)
        want = np.maximum(want, 0.0) if act == N.BCH_ACT_RELU else O.gelu_f64(want)
        assert O.max_rel_err(first, want) <= TOL, act
        for _ in range(2):
            assert np.array_equal(first, _sgemm_ex(dev, 1, x, w, b, act)), "not deterministic"


def test_sgemm_ex_transposed_split_groups_with_concurrent_work(dev):
    """The ring kernel's owners wait for blocks from other workgroups of the same launch (only
    lower-numbered ones, dispatched before them).  Run the decode calls while a second context's
    stream keeps every CU busy with 4096^3 GEMMs, so the ring kernel's workgroups are dispatched
    piecemeal as CUs free up: every result must equal the one from an idle device, bit for bit."""
    from barracuda_amd import HipDevice
    _say("sgemm_ex transposed split groups next to another stream's GEMMs")
    other = HipDevice()
    big = []  # the other context's tensors, released before it closes
    try:
        g = np.random.default_rng(3)
        big += [_up(other, g.standard_normal((4096, 4096), dtype=np.float32)) for _ in range(2)]
        big.append(Tensor.empty([4096, 4096], other))
        ba, bb, bc = big
        calls = []
        for i, (m, n, k) in enumerate(((8, 11008, 4096), (32, 11008, 4096), (8, 64, 16384))):
            rng = O.Lcg(40 + i)
            x, w, b = rng.normal((m, k)), rng.normal((n, k), 0.0, 0.05), rng.normal((n,))
            calls.append((m, n, k, _up(dev, x), _up(dev, w), _up(dev, b), Tensor.empty([m, n], dev)))

        def run(m, n, k, tx, tw, tb, ty):
            with dev._lock:
                dev.check(dev._lib.bch_sgemm_ex(dev.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr), k,
                                                C.c_void_p(tb.ptr), N.BCH_ACT_RELU, C.c_void_p(ty.ptr), n),
                          "sgemm_ex")

        want = []
        for c in calls:
            run(*c)
            want.append(c[-1].to_numpy())
        for _ in range(30):  # about 30 ms of work queued on the other stream, not waited for
            with other._lock:
                other.check(other._lib.bch_sgemm(other.ctx, 4096, 4096, 4096, C.c_void_p(ba.ptr), 4096,
                                                 C.c_void_p(bb.ptr), 4096, C.c_void_p(bc.ptr), 4096), "sgemm")
        for rep in range(10):
            for c, ref in zip(calls, want):
                run(*c)
                assert np.array_equal(c[-1].to_numpy(), ref), (rep, c[:3])
        other.sync()
    finally:
        ba = bb = bc = None
        big.clear()
        other.close()


def test_sgemm_ex_transposed_split_groups_exact_on_integers(dev):
    _say("sgemm_ex transposed split groups, integers")
    rng = np.random.default_rng(31)
    for m, n, k in ((8, 64, 16384), (32, 200, 2052), (5, 4096, 4096)):
        x = rng.integers(-8, 9, (m, k)).astype(np.float32)
        w = rng.integers(-8, 9, (n, k)).astype(np.float32)
        b = rng.integers(-100, 101, n).astype(np.float32)
        want = x.astype(np.int64) @ w.astype(np.int64).T + b
        assert np.array_equal(_sgemm_ex(dev, 1, x, w, b, N.BCH_ACT_NONE), want.astype(np.float32)), (m, n, k)


@pytest.mark.parametrize("m,n,k", [(1, 2048, 4096), (2, 2053, 2052), (3, 5000, 1024), (4, 4100, 6144),
                                   (4, 2304, 4100), (1, 3000, 44000), (6, 3000, 2048), (8, 11008, 4096),
                                   (5, 2053, 8196), (7, 4100, 100), (8, 40000, 512)])
def test_sgemm_ex_transposed_whole_rows(dev, m, n, k):
    """m <= 8, n >= 8 waves x CUs: each workgroup owns whole weight rows (one launch, no partials),
    its eight waves splitting K in passes of 4096.  Covers every row-block width (m = 1, 2, 3-4,
    5-8), rows per workgroup not a multiple of the transpose batch, K past a pass boundary (4100,
    6144, 8196: two and three passes, the last partial), K = 44000 (eleven passes), K = 100 (one
    live wave), and n = 40000 (more rows than one workgroup's LDS holds: more workgroups than
    CUs)."""
    _say(f"sgemm_ex transposed whole rows m={m} n={n} k={k}")
    rng = O.Lcg(m * 101 + n + 3 * k)
    x = rng.normal((m, k))
    w = rng.normal((n, k), 0.0, 0.05)
    bias = rng.normal((n,))
    for act, b in ((N.BCH_ACT_RELU, bias), (N.BCH_ACT_NONE, None)):
        got = _sgemm_ex(dev, 1, x, w, b, act)
        assert O.max_rel_err(got, _ref(x, w, b, True, act == N.BCH_ACT_RELU)) <= TOL, act
        assert np.array_equal(got, _sgemm_ex(dev, 1, x, w, b, act)), "not deterministic"


def test_sgemm_ex_transposed_whole_rows_exact_on_integers(dev):
    _say("sgemm_ex transposed whole rows, integers")
    rng = np.random.default_rng(23)
    for m, n, k in ((1, 2048, 96), (4, 2100, 2056), (2, 2048, 1024), (8, 2048, 4100), (6, 2100, 8192)):
        x = rng.integers(-8, 9, (m, k)).astype(np.float32)
        w = rng.integers(-8, 9, (n, k)).astype(np.float32)
        b = rng.integers(-100, 101, n).astype(np.float32)
        want = x.astype(np.int64) @ w.astype(np.int64).T + b
        assert np.array_equal(_sgemm_ex(dev, 1, x, w, b, N.BCH_ACT_NONE), want.astype(np.float32))


def test_sgemm_ex_transposed_unaligned_falls_back(dev):
    """lda not a multiple of 4: the tiled kernel's guarded path."""
    _say("sgemm_ex transposed unaligned lda")
    m, n, k = 8, 256, 130
    rng = O.Lcg(99)
    xp = rng.normal((m, k + 1))  # rows of k + 1 floats: lda = 131
    w = rng.normal((n, k), 0.0, 0.05)
    tx, tw = _up(dev, xp), _up(dev, w)
    ty = Tensor.empty([m, n], dev)
    with dev._lock:
        dev.check(dev._lib.bch_sgemm_ex(dev.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k + 1, C.c_void_p(tw.ptr), k, None,
                                        0, C.c_void_p(ty.ptr), n), "sgemm_ex")
    assert O.max_rel_err(ty.to_numpy(), _ref(np.ascontiguousarray(xp[:, :k]), w, None, True, False)) <= TOL


@pytest.mark.parametrize("transb", [0, 1])
def test_sgemm_ex_exact_on_integers(dev, transb):
    _say(f"sgemm_ex integers transb={transb}")
    rng = np.random.default_rng(17)
    for m, n, k in ((256, 256, 64), (4, 64, 96), (50, 70, 90)):
        x = rng.integers(-8, 9, (m, k)).astype(np.float32)
        w = rng.integers(-8, 9, (n, k) if transb else (k, n)).astype(np.float32)
        b = rng.integers(-100, 101, n).astype(np.float32)
        want = x.astype(np.int64) @ (w.astype(np.int64).T if transb else w.astype(np.int64)) + b
        got = _sgemm_ex(dev, transb, x, w, b, N.BCH_ACT_RELU)
        assert np.array_equal(got, np.maximum(want, 0).astype(np.float32))
        if transb:  # the reference's own f32 algorithm, bit for bit on integers
            assert np.array_equal(got, O.linear_f32(x, w, b, relu=True))


@pytest.mark.parametrize("m,n,k,transb", [(1024, 1024, 512, 1), (1024, 1024, 512, 0), (1000, 1024, 512, 1),
                                          (1001, 1003, 515, 0), (6144, 6144, 1536, 1)])
def test_epilogue_tile_gelu(dev, m, n, k, transb):
    """The 256 x 256 tile with the bias and activation epilogue (eight wavefronts, two per SIMD)
    in each load mode -- unguarded, float4-guarded, scalar-guarded -- and in the hybrid plan
    (6144^2 x 1536), with bias + GELU and bias + ReLU: one row from every 256-row tile against
    f64."""
    _say(f"epilogue tile m={m} n={n} k={k} transb={transb}")
    rng = O.Lcg(m + 5 * n + 3 * k + transb)
    x = rng.uniform((m, k))
    w = rng.uniform((n, k) if transb else (k, n))
    bias = rng.uniform((n,))
    rows = sorted({t * 256 + (t * 97 + 13) % 256 for t in range(m // 256)} | {0, m - 1})
    rows = [r for r in rows if r < m]
    z = _ref(x[rows], w, bias, transb, False)
    gelu = 0.5 * z * (1.0 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    for act, want in ((N.BCH_ACT_GELU, gelu), (N.BCH_ACT_RELU, np.maximum(z, 0.0))):
        got = _sgemm_ex(dev, transb, x, w, bias, act)[rows]
        assert O.max_rel_err(got, want) <= TOL, act


@pytest.mark.parametrize("batch,dims", [(256, [512, 1024, 256, 64]), (7, [33, 65, 17]), (1, [4096, 1024, 4096]),
                                        (1024, [256, 256, 256])])
def test_fused_mlp_vs_f64(dev, batch, dims):
    _say(f"fused_mlp batch={batch} dims={dims}")
    rng = O.Lcg(batch + sum(dims))
    x = rng.normal((batch, dims[0]))
    ws = [rng.normal((dims[i + 1], dims[i]), 0.0, 1.0 / np.sqrt(dims[i])) for i in range(len(dims) - 1)]
    bs = [rng.normal((dims[i + 1],), 0.0, 0.1) for i in range(len(dims) - 1)]
    got = fused_mlp(_up(dev, x), [_up(dev, w) for w in ws], [_up(dev, b) for b in bs], Activation.ReLU)
    assert got.shape() == [batch, dims[-1]]
    ref = O.fused_mlp_f64(x, ws, bs)
    assert O.max_rel_err(got.to_numpy(), ref) <= TOL
    if batch * max(dims) <= 1 << 20:
        assert O.max_rel_err(got.to_numpy(), O.fused_mlp_f32(x, ws, bs)) <= TOL


def test_fused_mlp_in_out_weights_and_square_layers(dev):
    """[in, out] weights are used as x W; square weights take the [out, in] reading (x W^T)."""
    _say("fused_mlp mixed weight orientation")
    rng = O.Lcg(23)
    x = rng.normal((64, 48))
    w0 = rng.normal((48, 80), 0.0, 0.15)   # [in, out] (48 != 80): x W
    w1 = rng.normal((80, 80), 0.0, 0.1)    # square: [out, in], x W^T
    w2 = rng.normal((10, 80), 0.0, 0.1)    # [out, in]
    bs = [rng.normal((80,)), rng.normal((80,)), rng.normal((10,))]
    got = fused_mlp(_up(dev, x), [_up(dev, w0), _up(dev, w1), _up(dev, w2)], [_up(dev, b) for b in bs])
    ref = O.fused_mlp_f64(x, [w0.T, w1, w2], bs)
    assert O.max_rel_err(got.to_numpy(), ref) <= TOL
