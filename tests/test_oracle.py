"""Pin the CPU oracle (oracle/bc_oracle.c) before trusting it.

Every oracle function is checked against something it does not compute
itself: the reference tests' literal vectors (tests/golden/), exact integer
arithmetic, closed forms, or brute force in numpy float64.  Planted-mistake
tests show the checks catch a transposed operand, a wrong scale, a flipped
mask and a changed summation order.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bc_oracle as O
from tests.conftest import case_inputs, f32

M64 = (1 << 64) - 1
MUL = 6364136223846793005
INC_MMIX = 1442695040888963407


# ---------------------------------------------------------------- generators
@pytest.mark.parametrize("seed", ["0", "1", "2", "3", "4", "42", "12345"])
def test_uniform_matches_exact_lcg(golden, seed):
    g = golden["lcg"][seed]
    got = O.Lcg(int(seed)).uniform(8)
    assert got.tolist() == g["uniform_pm1_f32"]
    u01 = O.Lcg(int(seed)).uniform(8, 0.0, 1.0)
    assert np.array_equal(u01, np.array(g["uniform_f64"], dtype=np.float32))


@pytest.mark.parametrize("seed", ["0", "1", "3", "4", "42"])
def test_normal_matches_box_muller(golden, seed):
    g = golden["lcg"][seed]
    got = O.Lcg(int(seed)).normal(8)
    want = np.array(g["normal_f64"], dtype=np.float32)
    # same f64 formula through the same libm: identical after rounding to f32
    assert np.array_equal(got, want)
    got3 = O.Lcg(int(seed)).normal(8, 0.0, 3.0)
    assert np.allclose(got3, np.float32(3.0) * want, rtol=1e-6, atol=0)


def test_jump_ahead_equals_stepping():
    for inc in (1, INC_MMIX):
        s = 987654321
        for n in (0, 1, 2, 7, 1000, 12345):
            x = s
            for _ in range(n):
                x = (x * MUL + inc) & M64
            assert O.lcg_advance(s, inc, n) == x


def test_parallel_fill_equals_sequential_stream():
    # the threaded fill must produce the exact sequential stream, and
    # filling A then B must continue the stream (argument order)
    n = 300_001
    rng = O.Lcg(7)
    a = rng.uniform(n)
    b = rng.uniform(5)
    s = 7
    idx = {0, 1, 2, n // 3, n // 2, n - 1}
    for i in range(n + 5):
        s = (s * MUL + 1) & M64
        if i in idx:
            assert a[i] == np.float32(2.0 * ((s >> 11) / float(1 << 53)) - 1.0)
        if i >= n:
            assert b[i - n] == np.float32(2.0 * ((s >> 11) / float(1 << 53)) - 1.0)
    # normals consume two draws each
    r2 = O.Lcg(11)
    x = r2.normal(1001)
    assert r2.state.value == O.lcg_advance(11, INC_MMIX, 2002)
    assert np.array_equal(x[:10], O.Lcg(11).normal(10))


def test_generator_moments():
    # ops/lattice/constants.rs tests: U(0,1) mean 0.5; N(0,1) mean ~0, var ~1
    u = O.Lcg(123).uniform(200_000, 0.0, 1.0).astype(np.float64)
    assert abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002
    z = O.Lcg(123).normal(200_000).astype(np.float64)
    assert abs(z.mean()) < 0.02 and abs(z.var() - 1.0) < 0.05
    assert u.min() >= 0.0 and u.max() < 1.0


# ---------------------------------------------------------------- matmul
def test_matmul_f64_golden(golden):
    for case in golden["matmul"]:
        a, b = case_inputs(case)
        got = O.matmul_f64(a, b).reshape(-1)
        want = np.array(case["expected"])
        # exact rational expected values; f64 accumulation of f32 products
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12), case["name"]


def test_matmul_f64_brute_force_and_row_selection():
    rng = np.random.default_rng(0)
    for (m, k, n) in [(1, 1, 1), (3, 5, 7), (17, 33, 9), (64, 3, 65)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        want = a.astype(np.longdouble) @ b.astype(np.longdouble)
        got = O.matmul_f64(a, b)
        assert np.allclose(got, want.astype(np.float64), rtol=1e-13, atol=1e-13)
        rows = [m - 1, 0]
        assert np.array_equal(O.matmul_f64(a, b, rows=rows), got[rows])


def test_matmul_f32_restatements_exact_on_integers():
    rng = np.random.default_rng(1)
    a = rng.integers(-8, 9, (37, 70)).astype(np.float32)
    b = rng.integers(-8, 9, (70, 45)).astype(np.float32)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(O.matmul_cpu_exec_f32(a, b), exact.astype(np.float32))
    assert np.array_equal(O.matmul_k1_f32(a, b), exact.astype(np.float32))
    bt = np.stack([a[:, :40].copy(), a[:, 30:].copy()])
    bb = np.stack([b[:40, :].copy(), b[30:, :].copy()])
    want = np.stack([a[:, :40].astype(np.int64) @ b[:40].astype(np.int64),
                     a[:, 30:].astype(np.int64) @ b[30:].astype(np.int64)])
    assert np.array_equal(O.batch_matmul_seq_f32(bt, bb), want.astype(np.float32))


def test_matmul_f32_restatements_within_tolerance_of_f64():
    rng = O.Lcg(2)
    a = rng.uniform((96, 512))
    b = rng.uniform((512, 80))
    ref = O.matmul_f64(a, b)
    for got in (O.matmul_cpu_exec_f32(a, b), O.matmul_k1_f32(a, b)):
        assert O.max_rel_err(got, ref) < 1e-5


def test_k1_order_differs_from_sequential_order():
    # pins the K1 grouping a0*b0 + (a1*b1 + (a2*b2 + (a3*b3 + acc))):
    # on [1, 1, 1e8, -1e8] sequential f32 accumulation loses the ones
    a = np.array([[1.0, 1.0, 1e8, -1e8]], dtype=np.float32)
    b = np.ones((4, 1), dtype=np.float32)
    assert O.matmul_cpu_exec_f32(a, b)[0, 0] == 0.0
    assert O.matmul_k1_f32(a, b)[0, 0] == 2.0
    assert O.matmul_f64(a, b)[0, 0] == 2.0


def test_planted_transposed_operand_fails_golden(golden):
    case = next(c for c in golden["matmul"] if c["name"] == "precision_2x3_3x2")
    a, b = case_inputs(case)
    wrong = O.matmul_f64(a, np.ascontiguousarray(b.reshape(2, 3).T))  # B read transposed
    assert not np.allclose(wrong.reshape(-1), case["expected"], atol=1e-5)


# ---------------------------------------------------------------- softmax
def test_softmax_golden(golden):
    for case in golden["softmax"]:
        x = np.array(case["x"], dtype=np.float32).reshape(case["shape"])
        axis = case.get("axis", len(case["shape"]) - 1)
        got32 = O.softmax_dim_f32(x, axis).reshape(-1)
        want = np.array(case["expected"])
        assert O.max_rel_err(got32, want) < 2e-7, case["name"]
        if axis == len(case["shape"]) - 1:
            got64 = O.softmax_rows_f64(x).reshape(-1)
            assert np.allclose(got64, want, rtol=1e-14, atol=1e-15), case["name"]
        if "sum_tol" in case:
            sums = got32.reshape(case["shape"]).sum(axis=axis)
            assert np.all(np.abs(sums - 1.0) < case["sum_tol"])
        if case.get("monotone"):
            assert np.all(np.diff(got32) > 0)
        if "last_gt" in case:
            assert got32[-1] > case["last_gt"]


def test_softmax_invariants_and_global():
    x = O.Lcg(1).normal((64, 300), 0.0, 3.0)
    y = O.softmax_rows_f64(x)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-14)
    # shift invariance and the all-equal row
    assert np.allclose(O.softmax_rows_f64(x + np.float32(5.0)), y, atol=1e-6)
    eq = np.full((2, 7), 3.0, dtype=np.float32)
    assert np.all(O.softmax_dim_f32(eq) == np.float32(1.0 / 7.0)) or \
        np.allclose(O.softmax_dim_f32(eq), 1.0 / 7.0, rtol=1e-7)
    g = O.softmax_global_f32(x)
    assert abs(float(g.astype(np.float64).sum()) - 1.0) < 1e-4
    # one sequential f32 sum over 19200 terms (the reference's order): its
    # rounding sets the elementwise relative error, ~1e-4 here
    ref = O.softmax_rows_f64(x.reshape(1, -1)).reshape(-1)
    assert np.max(np.abs(g.reshape(-1) - ref) / ref) < 1e-3


def test_softmax_axis_restatement_matches_transpose():
    x = O.Lcg(5).normal((3, 11, 6))
    got = O.softmax_dim_f32(x, 1)
    want = O.softmax_rows_f64(np.ascontiguousarray(np.moveaxis(x, 1, 2)))
    assert O.max_rel_err(got, np.ascontiguousarray(np.moveaxis(want, 2, 1))) < 1e-6


# ---------------------------------------------------------------- attention
def _np_sdpa(q, k, v, causal, scale):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if causal:
        i = np.arange(s.shape[2])[:, None]
        j = np.arange(s.shape[3])[None, :]
        s = np.where(j <= i, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, v)


def _att_inputs(case):
    sq = case.get("shape_q", case.get("shape"))
    skv = case.get("shape_kv", case.get("shape"))
    q = np.array(case["q"], dtype=np.float32).reshape(sq)
    k = np.array(case["k"], dtype=np.float32).reshape(skv)
    v = np.array(case["v"], dtype=np.float32).reshape(skv)
    return q, k, v


def test_sdpa_f64_closed_forms(golden):
    for case in golden["attention"]:
        q, k, v = _att_inputs(case)
        got = O.sdpa_f64(q, k, v, case["causal"]).reshape(-1)
        assert np.allclose(got, case["expected"], rtol=1e-12, atol=1e-12), case["name"]


def test_sdpa_f64_brute_force_cross_and_heads():
    rng = O.Lcg(4)
    for (B, H, Sq, Skv, D, causal) in [(1, 1, 5, 5, 3, True), (2, 3, 7, 7, 8, False),
                                        (1, 2, 4, 9, 16, False), (2, 2, 33, 33, 32, True)]:
        q = rng.normal((B, H, Sq, D))
        k = rng.normal((B, H, Skv, D))
        v = rng.normal((B, H, Skv, D))
        scale = 1.0 / math.sqrt(D)
        want = _np_sdpa(q, k, v, causal, scale)
        got = O.sdpa_f64(q, k, v, causal)
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
        heads = [B * H - 1, 0]
        sel = O.sdpa_f64(q, k, v, causal, heads=heads)
        assert np.array_equal(sel, got.reshape(B * H, Sq, D)[heads])
        # causal row 0 is exactly V[0]
        if causal:
            assert np.array_equal(got[:, :, 0, :], v[:, :, 0, :].astype(np.float64))


def test_attention_f32_restatements_within_tolerance():
    rng = O.Lcg(4)
    B, H, S, D = 1, 3, 64, 32
    q, k, v = rng.normal((B, H, S, D)), rng.normal((B, H, S, D)), rng.normal((B, H, S, D))
    for causal in (False, True):
        ref = O.sdpa_f64(q, k, v, causal)
        assert O.max_rel_err(O.attention_3pass_f32(q, k, v, causal), ref) < 1e-5
    ref = O.sdpa_f64(q, k, v, True)
    assert O.max_rel_err(O.causal_attention_cpu_f32(q, k, v), ref) < 1e-5
    # the CPU causal path on a head subset writes only those heads
    part = O.causal_attention_cpu_f32(q, k, v, 1, 2)
    assert np.array_equal(part[0, 1], O.causal_attention_cpu_f32(q, k, v)[0, 1])
    assert not part[0, 0].any() and not part[0, 2].any()


def test_planted_attention_mistakes_fail_closed_forms(golden):
    case = next(c for c in golden["attention"] if c["name"] == "causal_equal_scores_prefix_mean")
    q, k, v = _att_inputs(case)
    assert not np.allclose(O.sdpa_f64(q, k, v, False).reshape(-1), case["expected"], atol=1e-3)
    case = next(c for c in golden["attention"] if c["name"] == "one_hot_2x2")
    q, k, v = _att_inputs(case)
    assert not np.allclose(O.sdpa_f64(q, k, v, False, scale=1.0).reshape(-1), case["expected"], atol=1e-3)


# ---------------------------------------------------------------- metric
def test_max_rel_err_metric():
    ref = np.array([0.5, 10.0, -200.0], dtype=np.float64)
    x = np.array([0.5 + 1e-3, 10.0 + 1e-3, -200.0 - 2e-2], dtype=np.float32)
    # scale max(|ref|, 1): 1e-3/1, 1e-3/10, 2e-2/200
    assert abs(O.max_rel_err(x, ref) - 1e-3) < 1e-6
    assert O.max_rel_err(np.array([np.nan], np.float32), np.array([1.0])) == math.inf
    assert O.max_rel_err(np.array([np.inf], np.float32), np.array([np.inf])) == 0.0


def test_sdpa_f64_rows_equals_full_oracle_rows():
    """The row-sampled f64 attention oracle (used on all heads at config
    size) returns exactly the rows of the full oracle."""
    r = O.Lcg(5)
    q, k, v = (r.normal((2, 3, 40, 16)) for _ in range(3))
    rows = np.array([[0, 5, 39], [1, 2, 3], [39, 38, 0], [7, 7, 7], [10, 20, 30], [0, 1, 2]], dtype=np.int32)
    for causal in (False, True):
        full = O.sdpa_f64(q, k, v, causal).reshape(6, 40, 16)
        got = O.sdpa_f64_rows(q, k, v, causal, rows)
        assert np.array_equal(got, np.take_along_axis(full, rows[:, :, None].astype(np.int64), axis=1))


# ---- GELU and layer norm (session/mod.rs:349-398) --------------------------------
def test_gelu_oracle_reference_assertions_and_identities():
    """activations.rs:237-242 (GELU(0) = 0, GELU(10) > 9.99, |GELU(-10)| <
    0.01); the odd-part identity GELU(x) - GELU(-x) = x of the tanh form; the
    erf form x Phi(x) it approximates (tanh-form error below 5e-4 over
    [-8, 8]: a dropped cubic term is 0.034 off, a 0.04 coefficient 0.003)."""
    from scipy.special import erf
    g = O.gelu_f64(np.array([0.0, 10.0, -10.0], np.float32))
    assert g[0] == 0.0 and g[1] > 9.99 and abs(g[2]) < 0.01
    x = np.linspace(-8, 8, 40001).astype(np.float32)
    gx, gn = O.gelu_f64(x), O.gelu_f64(-x)
    xd = x.astype(np.float64)
    assert np.max(np.abs((gx - gn) - xd)) < 1e-12
    exact = 0.5 * xd * (1.0 + erf(xd / np.sqrt(2.0)))
    assert np.max(np.abs(gx - exact)) < 5e-4
    # large |x|: x and 0
    big = np.array([30.0, 1e4, -30.0, -1e4], np.float32)
    assert np.array_equal(O.gelu_f64(big), np.array([30.0, 1e4, -0.0, -0.0]))


def test_gelu_planted_mistakes_fail():
    from scipy.special import erf
    x = np.linspace(-8, 8, 4001)
    exact = 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))
    no_cubic = 0.5 * x * (1.0 + np.tanh(0.7978845608 * x))
    wrong_sign = 0.5 * x * (1.0 - np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))
    assert np.max(np.abs(no_cubic - exact)) > 5e-4
    assert np.max(np.abs(wrong_sign - exact)) > 5e-4


def test_gelu_f32_restatement_tracks_f64():
    x = O.Lcg(11).normal((100000,), 0.0, 4.0)
    assert O.max_rel_err(O.gelu_wgsl_f32(x), O.gelu_f64(x)) < 1e-6


def test_layer_norm_oracle_closed_forms():
    """layer_norm_f64.wgsl on [1,2,3,4]: mean 2.5, biased var 1.25 (an
    unbiased n-1 variance would be 5/3); the reference tests' vectors
    (ops/layer_norm_wgsl.rs:166-192: row means below 1e-5); output mean 0
    and biased variance var / (var + eps) on random rows; a constant row is
    0 (eps keeps 0 / sqrt(eps) finite); shift/scale invariance."""
    y = O.layer_norm_f64(np.array([[1, 2, 3, 4]], np.float32))
    want = (np.array([1, 2, 3, 4]) - 2.5) / np.sqrt(1.25 + 1e-5)
    assert np.max(np.abs(y[0] - want)) < 1e-12
    wrong = (np.array([1, 2, 3, 4]) - 2.5) / np.sqrt(5.0 / 3.0 + 1e-5)
    assert np.max(np.abs(y[0] - wrong)) > 1e-2
    y2 = O.layer_norm_f64(np.array([[1, 2, 3], [4, 5, 6]], np.float32))
    assert np.all(np.abs(y2.mean(axis=1)) < 1e-5)
    x = O.Lcg(12).normal((64, 777), 2.0, 3.0)
    y = O.layer_norm_f64(x, 1e-5)
    xd = x.astype(np.float64)
    v = xd.var(axis=1)
    assert np.max(np.abs(y.mean(axis=1))) < 1e-12
    assert np.max(np.abs(y.var(axis=1) - v / (v + 1e-5))) < 1e-12
    z = O.layer_norm_f64(np.full((2, 2048), 3.0, np.float32))
    assert np.array_equal(z, np.zeros((2, 2048)))
    # LN(a x) with eps a^2 equals LN(x) with eps (a = 4 is exact in f32), and
    # LN(x + b) = LN(x) on integer-valued rows (exact shifts)
    y_s = O.layer_norm_f64((x * np.float32(4.0)).astype(np.float32), 16e-5)
    assert np.max(np.abs(y_s - y)) < 1e-12
    xi = np.floor(O.Lcg(14).normal((8, 300), 0.0, 50.0)).astype(np.float32)
    assert np.max(np.abs(O.layer_norm_f64(xi + np.float32(1000.0)) - O.layer_norm_f64(xi))) < 1e-9


def test_layer_norm_f32_restatement_tracks_f64():
    x = O.Lcg(13).normal((256, 2048), 0.0, 3.0)
    assert O.max_rel_err(O.layer_norm_f32(x), O.layer_norm_f64(x)) < 1e-5


# ---------------------------------------------------------------- inline-data f64 handlers
def _ml_attention_longdouble(q, k, v, scale=True, subtract_max=True, v_t=False):
    """softmax(Q K^T / sqrt(d_k)) V in numpy longdouble, the mistakes below
    switchable (they are planted here, never in the oracle)."""
    q, k, v = (np.asarray(a, dtype=np.longdouble) for a in (q, k, v))
    s = q @ k.T
    if scale:
        s = s / np.sqrt(np.longdouble(q.shape[1]))
    if subtract_max:
        s = s - s.max(axis=1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=1, keepdims=True)
    return p @ (v.T if v_t else v)


def test_inline_f64_golden(golden):
    """sprint56b_tests.rs:618-669 and ml_tests.rs:128-165 through the oracle."""
    for case in golden["inline_f64"]:
        p = case["params"]
        if case["method"] == "tensor.matmul_inline":
            got = O.matmul_inline_f64(np.array(p["lhs"]), np.array(p["rhs"]))
        else:
            got = O.ml_attention_f64(np.array(p["q"]), np.array(p["k"]), np.array(p["v"]))
        want = np.array(case["expected"])
        assert got.shape == want.shape, case["name"]
        assert np.max(np.abs(got - want)) <= case["tol"] * max(1.0, np.max(np.abs(want))), case["name"]


def test_ml_softmax_rows_f64_closed_forms():
    y = O.ml_softmax_rows_f64(np.full((3, 8), 2.5))
    assert np.array_equal(y, np.full((3, 8), 0.125))               # equal row: exactly 1/8
    y = O.ml_softmax_rows_f64(np.array([[0.0, math.log(2.0)]]))
    assert np.max(np.abs(y - [[1 / 3, 2 / 3]])) < 1e-16
    x = O.Lcg(7).normal((5, 300)).astype(np.float64) * 30.0
    y = O.ml_softmax_rows_f64(x)
    assert np.all(np.abs(y.sum(axis=1) - 1.0) < 1e-14)
    assert np.max(np.abs(O.ml_softmax_rows_f64(x + 1000.0) - y)) < 1e-14  # shift invariance
    e = np.exp((x - x.max(axis=1, keepdims=True)).astype(np.longdouble))
    assert np.max(np.abs(y - (e / e.sum(axis=1, keepdims=True)).astype(np.float64))) < 1e-15
    # f64::max skips NaN, so the max is 2; exp(NaN - 2) poisons the sum: the row is NaN
    y = O.ml_softmax_rows_f64(np.array([[np.nan, 1.0, 2.0], [1000.0, 1001.0, 999.0]]))
    assert np.all(np.isnan(y[0]))
    assert np.all(np.isfinite(y[1])) and abs(y[1].sum() - 1.0) < 1e-15
    # a planted missing max subtraction overflows on that second row
    with np.errstate(over="ignore", invalid="ignore"):
        assert not np.all(np.isfinite(np.exp([1000.0, 1001.0]) / np.exp([1000.0, 1001.0]).sum()))


def test_ml_attention_f64_closed_forms_and_brute_force():
    # equal scores (q = 0): every row is the mean of the V rows
    v = np.arange(21, dtype=np.float64).reshape(7, 3) * 0.5
    out = O.ml_attention_f64(np.zeros((4, 5)), np.ones((7, 5)), v)
    assert np.max(np.abs(out - v.mean(axis=0))) < 1e-14
    rng = O.Lcg(11)
    for sq, sk, dk, dv in ((1, 1, 1, 1), (3, 5, 4, 2), (17, 33, 8, 17), (9, 9, 16, 9), (2, 300, 3, 7)):
        q, k, v = (rng.normal(s).astype(np.float64) for s in ((sq, dk), (sk, dk), (sk, dv)))
        got = O.ml_attention_f64(q, k, v)
        want = _ml_attention_longdouble(q, k, v).astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-13 * max(1.0, np.max(np.abs(want))), (sq, sk, dk, dv)


def test_ml_attention_planted_mistakes_fail():
    """A dropped scale, a transposed V and a missing max subtraction each
    fail the brute-force comparison that the oracle passes."""
    rng = O.Lcg(12)
    q, k, v = (rng.normal((9, 9)).astype(np.float64) * 3.0 for _ in range(3))
    good = O.ml_attention_f64(q, k, v)
    tol = 1e-13 * max(1.0, np.max(np.abs(good)))
    assert np.max(np.abs(good - _ml_attention_longdouble(q, k, v).astype(np.float64))) <= tol
    assert np.max(np.abs(good - _ml_attention_longdouble(q, k, v, scale=False).astype(np.float64))) > 1e-3
    assert np.max(np.abs(good - _ml_attention_longdouble(q, k, v, v_t=True).astype(np.float64))) > 1e-3
    big = q * 300.0  # scores of a few thousand: exp overflows f64 without the max subtraction
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(big @ k.T / 3.0)
        bad = (e / e.sum(axis=1, keepdims=True)) @ v
    ok = O.ml_attention_f64(big, k, v)
    assert np.all(np.isfinite(ok)) and not np.all(np.isfinite(bad))
    assert np.max(np.abs(ok - _ml_attention_longdouble(big, k, v).astype(np.float64))) <= 1e-12 * np.max(np.abs(ok))


def test_matmul_inline_f64_brute_force_and_planted_transpose():
    rng = O.Lcg(13)
    for m, k, n in ((1, 1, 1), (3, 7, 5), (16, 33, 9), (64, 64, 64)):
        a, b = rng.normal((m, k)).astype(np.float64), rng.normal((k, n)).astype(np.float64)
        got = O.matmul_inline_f64(a, b)
        want = (a.astype(np.longdouble) @ b.astype(np.longdouble)).astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-14 * max(1.0, np.max(np.abs(want))), (m, k, n)
    a, b = rng.normal((6, 6)).astype(np.float64), rng.normal((6, 6)).astype(np.float64)
    assert np.max(np.abs(O.matmul_inline_f64(a, b) - a @ b.T)) > 1e-3
    # integers: exact (fma chain of exact products and sums)
    ai = np.array(rng.uniform((8, 8), -50, 50), dtype=np.float64).round()
    bi = np.array(rng.uniform((8, 8), -50, 50), dtype=np.float64).round()
    assert np.array_equal(O.matmul_inline_f64(ai, bi), ai @ bi)
