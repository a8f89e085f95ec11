"""Seeded random parity sweep on the MI355X: shapes, leading dimensions, pointer offsets and
layouts drawn at random for each hot-path entry point, against the f64 oracle.

Entry points: bch_sgemm_ex, bch_sgemm_strided_batched, bch_dgemm, bch_sdpa_fwd_ex, bch_softmax_rows,
bch_softmax_axis, bch_layer_norm, bch_head_split and bch_head_concat.  The hand-picked tests
pin each kernel path at its boundaries; this sweep draws the arguments
those tests do not combine (odd leading dimensions with misaligned pointers, a transposed
weight with a bias and GELU at a decode shape, grouped heads in a padded sequence-major
layout at an odd head dimension, ...).  Every case is printed before it runs, and the seeds
are fixed, so a failure names its arguments.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against f64; padding
and the memory around each output must be left untouched.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from barracuda_amd import Tensor
from barracuda_amd import _native as N
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4
GUARD = 64  # floats of sentinel after every output


def _say(msg):
    print(msg, flush=True)


class _Buf:
    """A device buffer holding `data` (flat float32) at `off` floats in, with sentinels around."""

    def __init__(self, dev, data: np.ndarray, off: int):
        self.off, self.n = off, data.size
        host = np.full(off + data.size + GUARD, 7.25, np.float32)
        host[off:off + data.size] = data.reshape(-1)
        self.t = Tensor.from_data(host, [host.size], dev)
        self.ptr = C.c_void_p(self.t.ptr + 4 * off)

    def read(self) -> np.ndarray:
        return self.t.to_numpy().reshape(-1)

    def body(self) -> np.ndarray:
        return self.read()[self.off:self.off + self.n]

    def guards_intact(self) -> bool:
        h = self.read()
        return bool(np.all(h[:self.off] == 7.25) and np.all(h[self.off + self.n:] == 7.25))


def _gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def _gemm_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        m = int(rng.choice([rng.integers(1, 33), rng.integers(33, 65), rng.integers(65, 400)]))
        n = int(rng.integers(1, 700))
        k = int(rng.choice([rng.integers(1, 40), rng.integers(40, 800)]))
        yield dict(m=m, n=n, k=k, transb=int(rng.integers(0, 2)), pa=int(rng.choice([0, 0, 1, 3, 4])),
                   pb=int(rng.choice([0, 0, 1, 4])), pc=int(rng.choice([0, 0, 2, 4])),
                   oa=int(rng.choice([0, 0, 1])), ob=int(rng.choice([0, 0, 3])), oc=int(rng.choice([0, 0, 1])),
                   bias=bool(rng.integers(0, 2)), act=int(rng.integers(0, 3)))


def _gemm64_cases(n_cases: int, seed: int):
    """Multiples of 64 up to 1024: the 64 x 64 x 64 tiles where the leading dimensions and
    pointers allow, split-K or the usual tiles where they do not."""
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        yield dict(m=64 * int(rng.integers(1, 17)), n=64 * int(rng.integers(1, 17)), k=64 * int(rng.integers(1, 17)),
                   transb=int(rng.integers(0, 2)), pa=int(rng.choice([0, 0, 4, 1])), pb=int(rng.choice([0, 0, 8, 3])),
                   pc=int(rng.choice([0, 0, 4])), oa=int(rng.choice([0, 0, 0, 1])), ob=int(rng.choice([0, 0, 4])),
                   oc=int(rng.choice([0, 0, 1])), bias=bool(rng.integers(0, 2)), act=int(rng.integers(0, 3)))


@pytest.mark.parametrize("case", list(_gemm_cases(150, 2026)), ids=lambda c: "m{m}n{n}k{k}t{transb}".format(**c))
def test_sgemm_ex_random(dev, case):
    """bch_sgemm_ex: C = act(A op(B) + bias) with padded leading dimensions and misaligned
    pointers, every kernel family (skinny, two-block skinny, tiles, split-K, hybrid)."""
    _check_sgemm_ex(dev, case)


@pytest.mark.parametrize("case", list(_gemm64_cases(40, 6464)), ids=lambda c: "m{m}n{n}k{k}t{transb}".format(**c))
def test_sgemm_ex_random_multiples_of_64(dev, case):
    """bch_sgemm_ex at shapes in multiples of 64 (the small tiles' domain) with the same
    random padding, offsets, bias and activation."""
    _check_sgemm_ex(dev, case)


def _check_sgemm_ex(dev, case):
    _say(f"sgemm_ex random {case} ({dev._lib.bch_sgemm_kernel_name(case['m'], case['n'], case['k']).decode()})")
    m, n, k, tb = case["m"], case["n"], case["k"], case["transb"]
    rng = np.random.default_rng(m * 1000003 + n * 1009 + k)
    lda, ldc = k + case["pa"], n + case["pc"]
    ldb = (k if tb else n) + case["pb"]
    a = rng.standard_normal((m, k)).astype(np.float32)
    bmat = (rng.standard_normal((k, n)) / math.sqrt(max(k, 1))).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) if case["bias"] else None
    ah = np.zeros((m, lda), np.float32)
    ah[:, :k] = a
    stored_b = bmat.T if tb else bmat
    bh = np.zeros((stored_b.shape[0], ldb), np.float32)
    bh[:, :stored_b.shape[1]] = stored_b
    ch = np.full((m, ldc), -3.5, np.float32)
    A, B, Cb = _Buf(dev, ah, case["oa"]), _Buf(dev, bh, case["ob"]), _Buf(dev, ch, case["oc"])
    Bias = _Buf(dev, bias, 0) if bias is not None else None
    lib = dev._lib
    dev.check(lib.bch_sgemm_ex(dev.ctx, tb, m, n, k, A.ptr, lda, B.ptr, ldb, Bias.ptr if Bias else None,
                               case["act"], Cb.ptr, ldc), "sgemm_ex")
    got = Cb.body().reshape(m, ldc)
    ref = a.astype(np.float64) @ bmat.astype(np.float64)
    if bias is not None:
        ref = ref + bias.astype(np.float64)
    if case["act"] == 1:
        ref = np.maximum(ref, 0.0)
    elif case["act"] == 2:
        ref = _gelu64(ref)
    assert O.max_rel_err(np.ascontiguousarray(got[:, :n]), ref) <= TOL
    assert np.all(got[:, n:] == -3.5), "padding columns of C written"
    assert Cb.guards_intact() and A.guards_intact() and B.guards_intact()


def _dgemm_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        yield dict(batch=int(rng.integers(1, 4)), m=int(rng.choice([rng.integers(1, 140), 2 * rng.integers(64, 160)])),
                   n=int(rng.choice([rng.integers(1, 140), 2 * rng.integers(64, 160)])),
                   k=int(rng.choice([rng.integers(1, 64), 2 * rng.integers(32, 700)])),
                   ta=int(rng.integers(0, 2)), tb=int(rng.integers(0, 2)), pa=int(rng.choice([0, 0, 2, 1])),
                   pb=int(rng.choice([0, 0, 2, 3])), pc=int(rng.choice([0, 0, 1])), ga=int(rng.choice([0, 0, 2, 1])),
                   gb=int(rng.choice([0, 0, 4])), gc=int(rng.choice([0, 0, 3])), oa=int(rng.choice([0, 0, 0, 1])),
                   ob=int(rng.choice([0, 0, 2])), alpha=float(rng.choice([1.0, -0.75])),
                   beta=float(rng.choice([0.0, 0.0, 1.5])))


@pytest.mark.parametrize("case", list(_dgemm_cases(60, 6402)),
                         ids=lambda c: "b{batch}m{m}n{n}k{k}t{ta}{tb}".format(**c))
def test_dgemm_random(dev, case):
    """bch_dgemm: C = alpha op(A) op(B) (+ beta C) with padded leading dimensions, gaps between
    batches and operands 8 bytes off 16-byte alignment; the pair-guarded and scalar-guarded
    tiles, split k.  Against a longdouble product within 1e-12; padding and the memory around C
    are left alone."""
    _say(f"dgemm random {case}")
    from barracuda_amd import F64Buffer
    bt, m, n, k, ta, tb = case["batch"], case["m"], case["n"], case["k"], case["ta"], case["tb"]
    rng = np.random.default_rng(bt * 7 + m * 1009 + n * 31 + k + 2 * ta + tb)
    ar, ac = (k, m) if ta else (m, k)  # stored A rows x cols
    br, bc = (n, k) if tb else (k, n)
    lda, ldb, ldc = ac + case["pa"], bc + case["pb"], n + case["pc"]
    sA, sB, sC = ar * lda + case["ga"], br * ldb + case["gb"], m * ldc + case["gc"]
    a = rng.uniform(-1, 1, (bt, ar, ac))
    b = rng.uniform(-1, 1, (bt, br, bc))
    c0 = rng.uniform(-1, 1, (bt, m, n))
    A = np.full(case["oa"] + bt * sA + 8, 7.25)
    B = np.full(case["ob"] + bt * sB + 8, 7.25)
    Cb = np.full(bt * sC + 8, 7.25)
    for z in range(bt):
        A[case["oa"] + z * sA:case["oa"] + z * sA + ar * lda].reshape(ar, lda)[:, :ac] = a[z]
        B[case["ob"] + z * sB:case["ob"] + z * sB + br * ldb].reshape(br, ldb)[:, :bc] = b[z]
        Cb[z * sC:z * sC + m * ldc].reshape(m, ldc)[:, :n] = c0[z]
    da, db, dc = (F64Buffer(dev, x.size).upload(x) for x in (A, B, Cb))
    with dev._lock:
        dev.check(dev._lib.bch_dgemm(dev.ctx, ta, tb, bt, m, n, k, case["alpha"], C.c_void_p(da.ptr + 8 * case["oa"]),
                                     lda, sA, C.c_void_p(db.ptr + 8 * case["ob"]), ldb, sB, case["beta"],
                                     C.c_void_p(dc.ptr), ldc, sC), "dgemm")
    out = dc.to_vec()
    for z in range(bt):
        opa = a[z].astype(np.longdouble).T if ta else a[z].astype(np.longdouble)
        opb = b[z].astype(np.longdouble).T if tb else b[z].astype(np.longdouble)
        ref = case["alpha"] * (opa @ opb)
        if case["beta"] != 0.0:
            ref = ref + case["beta"] * c0[z].astype(np.longdouble)
        blk = out[z * sC:z * sC + m * ldc].reshape(m, ldc)
        err = float(np.max(np.abs(blk[:, :n] - ref.astype(np.float64)) / np.maximum(np.abs(ref.astype(np.float64)), 1.0)))
        assert err <= 1e-12, (z, err)
        keep = Cb[z * sC:z * sC + m * ldc].reshape(m, ldc)[:, n:]
        assert np.array_equal(blk[:, n:], keep), "padding columns of C written"
        assert np.all(out[z * sC + m * ldc:(z + 1) * sC] == 7.25), "gap between batches written"
    assert np.all(out[bt * sC:] == 7.25), "memory after C written"


def _batched_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        yield dict(batch=int(rng.integers(1, 6)), m=int(rng.integers(1, 300)), n=int(rng.integers(1, 300)),
                   k=int(rng.integers(1, 300)), ga=int(rng.choice([0, 0, 5])), gb=int(rng.choice([0, 0, 8])),
                   gc=int(rng.choice([0, 0, 3])))


@pytest.mark.parametrize("case", list(_batched_cases(40, 77)), ids=lambda c: "b{batch}m{m}n{n}k{k}".format(**c))
def test_sgemm_strided_batched_random(dev, case):
    """bch_sgemm_strided_batched with gaps between the batches (strides above the dense ones)."""
    _say(f"sgemm batched random {case}")
    bt, m, n, k = case["batch"], case["m"], case["n"], case["k"]
    sa, sb, sc = m * k + case["ga"], k * n + case["gb"], m * n + case["gc"]
    rng = np.random.default_rng(bt * 7919 + m * 131 + n * 17 + k)
    a = rng.standard_normal((bt, m, k)).astype(np.float32)
    b = rng.standard_normal((bt, k, n)).astype(np.float32)
    ah, bh = np.zeros(bt * sa, np.float32), np.zeros(bt * sb, np.float32)
    for i in range(bt):
        ah[i * sa:i * sa + m * k] = a[i].reshape(-1)
        bh[i * sb:i * sb + k * n] = b[i].reshape(-1)
    A, B, Cb = _Buf(dev, ah, 0), _Buf(dev, bh, 0), _Buf(dev, np.full(bt * sc, -3.5, np.float32), 0)
    dev.check(dev._lib.bch_sgemm_strided_batched(dev.ctx, bt, m, n, k, A.ptr, sa, B.ptr, sb, Cb.ptr, sc), "batched")
    out = Cb.body()
    for i in range(bt):
        got = out[i * sc:i * sc + m * n].reshape(m, n)
        assert O.max_rel_err(got, a[i].astype(np.float64) @ b[i].astype(np.float64)) <= TOL, i
        assert np.all(out[i * sc + m * n:(i + 1) * sc] == -3.5), "gap between batches written"
    assert Cb.guards_intact()


def _attn_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        hkv = int(rng.integers(1, 4))
        g = int(rng.integers(1, 4))
        causal = bool(rng.integers(0, 2))
        sq = int(rng.integers(1, 260))
        skv = sq if causal else int(rng.integers(1, 260))
        d = int(rng.choice([rng.integers(1, 129), rng.integers(129, 257), rng.integers(257, 400)]))
        yield dict(B=int(rng.integers(1, 3)), H=hkv * g, Hkv=hkv, Sq=sq, Skv=skv, D=d, causal=causal,
                   qlay=str(rng.choice(["bhsd", "bshd"])), olay=str(rng.choice(["bhsd", "bshd"])),
                   pad=int(rng.choice([0, 0, 4, 3])))


def _place(x: np.ndarray, lay: str, pad: int):
    """x [B, H, S, D] stored in layout lay ('bhsd' dense, or 'bshd' with rows of H*D + pad
    floats); returns (flat array, (batch, head, row) strides)."""
    Bn, Hn, Sn, Dn = x.shape
    if lay == "bhsd":
        return x.reshape(-1).copy(), (Hn * Sn * Dn, Sn * Dn, Dn)
    row = Hn * Dn + pad
    flat = np.zeros((Bn, Sn, row), np.float32)
    flat[:, :, :Hn * Dn] = x.transpose(0, 2, 1, 3).reshape(Bn, Sn, Hn * Dn)
    return flat.reshape(-1), (Sn * row, Dn, row)


def _gather(flat: np.ndarray, st, shape):
    Bn, Hn, Sn, Dn = shape
    idx = (np.arange(Bn)[:, None, None, None] * st[0] + np.arange(Hn)[None, :, None, None] * st[1]
           + np.arange(Sn)[None, None, :, None] * st[2] + np.arange(Dn)[None, None, None, :])
    return flat[idx]


@pytest.mark.parametrize("case", list(_attn_cases(100, 4242)),
                         ids=lambda c: "B{B}H{H}kv{Hkv}q{Sq}k{Skv}D{D}c{causal:d}".format(**c))
def test_sdpa_ex_random(dev, case):
    """bch_sdpa_fwd_ex: grouped key/value heads, Q and O in dense or padded sequence-major
    layouts, head dimensions across the fused kernels (<= 128, <= 256) and the chunked path."""
    _say(f"sdpa_ex random {case}")
    Bn, H, Hkv, Sq, Skv, D = (case[x] for x in ("B", "H", "Hkv", "Sq", "Skv", "D"))
    rng = np.random.default_rng(Bn * 31 + H * 7 + Sq * 3 + Skv * 5 + D)
    q = rng.standard_normal((Bn, H, Sq, D)).astype(np.float32)
    k = rng.standard_normal((Bn, Hkv, Skv, D)).astype(np.float32)
    v = rng.standard_normal((Bn, Hkv, Skv, D)).astype(np.float32)
    qf, qs = _place(q, case["qlay"], case["pad"])
    kf, ks = _place(k, "bhsd", 0)
    vf, vs = _place(v, "bhsd", 0)
    of, os_ = _place(np.zeros((Bn, H, Sq, D), np.float32), case["olay"], case["pad"])
    of[:] = -3.5
    Q, K, V, Ob = _Buf(dev, qf, 0), _Buf(dev, kf, 1), _Buf(dev, vf, 0), _Buf(dev, of, 0)
    scale = float(np.float32(1) / np.sqrt(np.float32(D)))
    dev.check(dev._lib.bch_sdpa_fwd_ex(dev.ctx, Bn, H, Hkv, Sq, Skv, D, scale, int(case["causal"]), Q.ptr,
                                       N.AttnLayout(*qs), K.ptr, N.AttnLayout(*ks), V.ptr, N.AttnLayout(*vs),
                                       Ob.ptr, N.AttnLayout(*os_)), "sdpa_fwd_ex")
    flat = Ob.body()
    got = _gather(flat, os_, (Bn, H, Sq, D))
    assert O.max_rel_err(np.ascontiguousarray(got), O.gqa_f64(q, k, v, case["causal"])) <= TOL
    touched = np.zeros(flat.size, bool)
    touched[_gather(np.arange(flat.size), os_, (Bn, H, Sq, D)).reshape(-1)] = True
    assert np.all(flat[~touched] == -3.5), "padding of O written"
    assert Ob.guards_intact()


def _softmax_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        if rng.integers(0, 2):
            cols = int(rng.choice([rng.integers(1, 5000), rng.integers(5000, 70000), rng.integers(70000, 300000)]))
            rows = int(rng.integers(1, max(2, min(3000, 3_000_000 // cols))))
            yield dict(kind="rows", outer=rows, axis=cols, inner=1, off=int(rng.choice([0, 0, 1, 2])),
                       inplace=bool(rng.integers(0, 2)))
        else:
            inner = int(rng.choice([rng.integers(2, 17), rng.integers(17, 300), rng.integers(1000, 2100)]))
            axis = int(rng.integers(1, max(2, min(40000, 3_000_000 // inner))))
            outer = int(rng.integers(1, max(2, min(8, 3_000_000 // (inner * axis)))))
            yield dict(kind="axis", outer=outer, axis=axis, inner=inner, off=int(rng.choice([0, 0, 1])),
                       inplace=bool(rng.integers(0, 2)))


@pytest.mark.parametrize("case", list(_softmax_cases(100, 99)),
                         ids=lambda c: "{kind}{outer}x{axis}x{inner}".format(**c))
def test_softmax_random(dev, case):
    """bch_softmax_rows / bch_softmax_axis at random shapes, offsets and in place."""
    _say(f"softmax random {case}")
    o, a, i = case["outer"], case["axis"], case["inner"]
    x = O.Lcg(o * 7 + a * 3 + i).normal((o, a, i), 0.0, 3.0)
    X = _Buf(dev, x, case["off"])
    Y = X if case["inplace"] else _Buf(dev, np.full(x.size, -3.5, np.float32), case["off"] ^ 1)
    lib = dev._lib
    if case["kind"] == "rows":
        dev.check(lib.bch_softmax_rows(dev.ctx, o, a, X.ptr, Y.ptr), "rows")
    else:
        dev.check(lib.bch_softmax_axis(dev.ctx, o, a, i, X.ptr, Y.ptr), "axis")
    got = Y.body().reshape(o, a, i)
    want = np.moveaxis(O.softmax_rows_f64(np.ascontiguousarray(np.moveaxis(x, 1, -1))), -1, 1)
    assert O.max_rel_err(np.ascontiguousarray(got), np.ascontiguousarray(want)) <= TOL
    assert Y.guards_intact() and X.guards_intact()


def _norm_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        cols = int(rng.choice([rng.integers(1, 4100), rng.integers(4100, 70000), rng.integers(70000, 200000)]))
        rows = int(rng.integers(1, max(2, min(2000, 2_000_000 // cols))))
        yield dict(rows=rows, cols=cols, off=int(rng.choice([0, 0, 1, 3])), inplace=bool(rng.integers(0, 2)))


@pytest.mark.parametrize("case", list(_norm_cases(60, 5)), ids=lambda c: "{rows}x{cols}".format(**c))
def test_layer_norm_random(dev, case):
    """bch_layer_norm (TensorSession::layer_norm, layer_norm_f64.wgsl) at random shapes, offsets
    and in place."""
    _say(f"layer_norm random {case}")
    r, c = case["rows"], case["cols"]
    x = O.Lcg(r * 11 + c).normal((r, c), 0.5, 2.0)
    X = _Buf(dev, x, case["off"])
    Y = X if case["inplace"] else _Buf(dev, np.full(x.size, -3.5, np.float32), case["off"] ^ 1)
    dev.check(dev._lib.bch_layer_norm(dev.ctx, r, c, 1e-5, X.ptr, Y.ptr), "layer_norm")
    assert O.max_rel_err(Y.body().reshape(r, c), O.layer_norm_f64(x)) <= TOL
    assert Y.guards_intact() and X.guards_intact()


def _perm_cases(n_cases: int, seed: int):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        yield dict(B=int(rng.integers(1, 4)), S=int(rng.integers(1, 300)), H=int(rng.integers(1, 17)),
                   D=int(rng.choice([rng.integers(1, 9), rng.integers(9, 200)])), concat=bool(rng.integers(0, 2)),
                   oi=int(rng.choice([0, 0, 1])), oo=int(rng.choice([0, 0, 2])))


@pytest.mark.parametrize("case", list(_perm_cases(60, 8)), ids=lambda c: "B{B}S{S}H{H}D{D}c{concat:d}".format(**c))
def test_head_permute_random(dev, case):
    """bch_head_split / bch_head_concat, bit-exact against numpy's transpose, with misaligned
    pointers (the scalar path) among them."""
    _say(f"head permute random {case}")
    Bn, S, H, D = case["B"], case["S"], case["H"], case["D"]
    rng = np.random.default_rng(Bn * 1009 + S * 31 + H * 7 + D)
    if case["concat"]:
        x = rng.standard_normal((Bn, H, S, D)).astype(np.float32)
        want = x.transpose(0, 2, 1, 3).reshape(-1)
        fn = dev._lib.bch_head_concat
    else:
        x = rng.standard_normal((Bn, S, H * D)).astype(np.float32)
        want = x.reshape(Bn, S, H, D).transpose(0, 2, 1, 3).reshape(-1)
        fn = dev._lib.bch_head_split
    X, Y = _Buf(dev, x, case["oi"]), _Buf(dev, np.full(x.size, -3.5, np.float32), case["oo"])
    dev.check(fn(dev.ctx, Bn, S, H, D, X.ptr, Y.ptr), "head_permute")
    assert np.array_equal(Y.body(), want)
    assert Y.guards_intact() and X.guards_intact()
