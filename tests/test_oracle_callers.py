"""Pin the oracle of the attention callers (grouped-query and multi-head
attention) and test their host-side validation, all on the CPU.

Checks use what the oracle does not compute itself: the reference tests'
inputs with their closed-form outputs, brute-force loops that index heads
explicitly, and planted mistakes (a wrong key/value head map, an interleaved
head split) that must fail.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from barracuda_amd import (DeviceError, GroupedQueryAttention, InvalidInput, InvalidOperation,
                           MultiHeadAttention, ShapeMismatch, Tensor)
from oracle import bc_oracle as O


def _brute_attention(q, k, v, causal=False):
    """numpy float64 loops over one (query row, key) pair at a time."""
    sq, d = q.shape
    out = np.zeros((sq, v.shape[1]))
    for i in range(sq):
        n = i + 1 if causal else k.shape[0]
        s = np.array([float(np.dot(q[i].astype(np.float64), k[j].astype(np.float64))) for j in range(n)])
        s /= math.sqrt(d)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[i] = p @ v[:n].astype(np.float64)
    return out


# ------------------------------------------------------------------ GQA
def test_gqa_oracle_reference_vector():
    # ops/grouped_query_attention/tests.rs:21-38: Q [1,8,4,4], K/V [1,2,4,4], all 0.5;
    # equal scores -> uniform weights -> the mean of V rows = 0.5
    q = np.full((1, 8, 4, 4), 0.5, np.float32)
    kv = np.full((1, 2, 4, 4), 0.5, np.float32)
    assert np.array_equal(O.gqa_f64(q, kv, kv), np.full((1, 8, 4, 4), 0.5))
    assert np.array_equal(O.gqa_3pass_f32(q, kv, kv), np.full((1, 8, 4, 4), 0.5, np.float32))


@pytest.mark.parametrize("causal", [False, True])
def test_gqa_oracle_brute_force_and_planted_head_map(causal):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, S, D = 2, 6, 2, 5, 3
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    got = O.gqa_f64(q, k, v, causal)
    want = np.empty_like(got)
    wrong = np.empty_like(got)
    for b in range(B):
        for h in range(Hq):
            want[b, h] = _brute_attention(q[b, h], k[b, h // 3], v[b, h // 3], causal)  # heads_per_group 3
            wrong[b, h] = _brute_attention(q[b, h], k[b, h % Hkv], v[b, h % Hkv], causal)
    assert np.max(np.abs(got - want)) < 1e-12
    assert np.max(np.abs(got - wrong)) > 1e-2  # a modulo head map is caught
    if not causal:
        f32 = O.gqa_3pass_f32(q, k, v)
        assert O.max_rel_err(f32, want) < 1e-5


# ------------------------------------------------------------------ MHA
@pytest.mark.parametrize("sq,skv", [(8, 8), (8, 16)])
def test_mha_oracle_reference_vectors(sq, skv):
    # ops/mha/tests.rs:9-56 (basic) and :98-149 (cross-attention): B 2, d_model 64, 8 heads,
    # q = k = 0.5, v = 1.0, every weight 0.01.  Projections: 0.5*0.01*64 = 0.32 (q, k) and
    # 0.64 (v); equal scores -> each head's output is 0.64; out = 0.64 * 0.01 * 64 = 0.4096.
    q = np.full((2, sq, 64), 0.5, np.float32)
    k = np.full((2, skv, 64), 0.5, np.float32)
    v = np.full((2, skv, 64), 1.0, np.float32)
    w = np.full((64, 64), 0.01, np.float32)
    got = O.mha_f64(q, k, v, w, w, w, w, 8)
    w64 = float(np.float32(0.01))
    assert got.shape == (2, sq, 64)
    assert np.allclose(got, (1.0 * w64 * 64) * w64 * 64, rtol=0, atol=1e-15)


def test_mha_oracle_one_head_identity_weights_is_attention():
    rng = np.random.default_rng(3)
    B, S, D = 2, 7, 5
    q, k, v = (rng.standard_normal((B, S, D)).astype(np.float32) for _ in range(3))
    eye = np.eye(D, dtype=np.float32)
    got = O.mha_f64(q, k, v, eye, eye, eye, eye, 1)
    want = O.sdpa_f64(q[:, None], k[:, None], v[:, None], False)[:, 0]
    assert np.max(np.abs(got - want)) < 1e-12


def test_mha_oracle_brute_force_and_planted_head_split():
    rng = np.random.default_rng(11)
    B, Sq, Skv, D, H = 2, 4, 6, 12, 3
    hd = D // H
    q = rng.standard_normal((B, Sq, D)).astype(np.float32)
    k, v = (rng.standard_normal((B, Skv, D)).astype(np.float32) for _ in range(2))
    wq, wk, wv, wo = (rng.standard_normal((D, D)).astype(np.float32) / 3 for _ in range(4))
    got = O.mha_f64(q, k, v, wq, wk, wv, wo, H)

    def run(cols):
        out = np.zeros((B, Sq, D))
        for b in range(B):
            qp = q[b].astype(np.float64) @ wq
            kp = k[b].astype(np.float64) @ wk
            vp = v[b].astype(np.float64) @ wv
            o = np.zeros((Sq, D))
            for h in range(H):
                c = cols(h)
                o[:, c] = _brute_attention(qp[:, c], kp[:, c], vp[:, c])
            out[b] = o @ wo
        return out

    want = run(lambda h: slice(h * hd, (h + 1) * hd))          # head h = columns h*hd .. h*hd+hd-1
    wrong = run(lambda h: slice(h, D, H))                        # interleaved columns
    assert np.max(np.abs(got - want)) < 1e-10
    assert np.max(np.abs(got - wrong)) > 1e-3


# ------------------------------------------------------------------ host validation (no device use)
def _t(shape, dev):
    return Tensor(None, shape, dev)


def test_gqa_validation_mirrors_reference():
    dev = object()
    with pytest.raises(InvalidInput, match="4D tensors"):
        GroupedQueryAttention(_t([1, 8, 4], dev), _t([1, 2, 4, 4], dev), _t([1, 2, 4, 4], dev))
    with pytest.raises(ShapeMismatch):
        GroupedQueryAttention(_t([1, 8, 4, 4], dev), _t([1, 2, 5, 4], dev), _t([1, 2, 5, 4], dev))
    with pytest.raises(ShapeMismatch):
        GroupedQueryAttention(_t([1, 8, 4, 4], dev), _t([1, 2, 4, 4], dev), _t([1, 4, 4, 4], dev))
    with pytest.raises(InvalidInput, match=r"num_q_heads \(8\) must be divisible by num_kv_heads \(3\)"):
        GroupedQueryAttention(_t([1, 8, 4, 4], dev), _t([1, 3, 4, 4], dev), _t([1, 3, 4, 4], dev))
    with pytest.raises(DeviceError):
        GroupedQueryAttention(_t([1, 8, 4, 4], dev), _t([1, 2, 4, 4], object()), _t([1, 2, 4, 4], dev))
    GroupedQueryAttention(_t([1, 8, 4, 4], dev), _t([1, 2, 4, 4], dev), _t([1, 2, 4, 4], dev))


def test_mha_validation_mirrors_reference():
    dev = object()
    x, w = _t([2, 8, 64], dev), _t([64, 64], dev)
    with pytest.raises(ShapeMismatch):
        MultiHeadAttention(_t([16, 64], dev), x, x, w, w, w, w, 8)
    with pytest.raises(ShapeMismatch):
        MultiHeadAttention(x, _t([3, 8, 64], dev), _t([3, 8, 64], dev), w, w, w, w, 8)
    with pytest.raises(ShapeMismatch):
        MultiHeadAttention(x, _t([2, 8, 32], dev), _t([2, 8, 32], dev), w, w, w, w, 8)
    with pytest.raises(ShapeMismatch):
        MultiHeadAttention(x, _t([2, 16, 64], dev), _t([2, 8, 64], dev), w, w, w, w, 8)
    with pytest.raises(ShapeMismatch):
        MultiHeadAttention(x, x, x, _t([64, 32], dev), w, w, w, 8)
    # tests.rs:59-96: d_model 64 with 7 heads is an error
    with pytest.raises(InvalidOperation, match=r"d_model \(64\) must be divisible by num_heads \(7\)"):
        MultiHeadAttention(x, x, x, w, w, w, w, 7)
    MultiHeadAttention(x, x, x, w, w, w, w, 8)
    # cross-attention: query and key/value sequence lengths may differ
    MultiHeadAttention(x, _t([2, 16, 64], dev), _t([2, 16, 64], dev), w, w, w, w, 8)


def test_reshape_is_a_view_with_the_same_element_count():
    dev = object()
    t = _t([2, 8, 64], dev)
    assert t.reshape([16, 64]).shape() == [16, 64]
    with pytest.raises(ShapeMismatch):
        t.reshape([15, 64])


# ------------------------------------------------------------------ linear / fused MLP
def test_linear_f32_exact_on_integers():
    rng = np.random.default_rng(5)
    x = rng.integers(-8, 9, (6, 13)).astype(np.float32)
    w = rng.integers(-8, 9, (9, 13)).astype(np.float32)  # [out, in]
    b = rng.integers(-50, 51, 9).astype(np.float32)
    want = x.astype(np.int64) @ w.astype(np.int64).T + b.astype(np.int64)
    assert np.array_equal(O.linear_f32(x, w, b), want.astype(np.float32))
    assert np.array_equal(O.linear_f32(x, w, b, relu=True), np.maximum(want, 0).astype(np.float32))
    assert np.array_equal(O.linear_f32(x, w), (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


def test_fused_mlp_oracles_agree_and_closed_forms():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 12)).astype(np.float32)
    ws = [rng.standard_normal((16, 12)).astype(np.float32) / 3, rng.standard_normal((7, 16)).astype(np.float32) / 4]
    bs = [rng.standard_normal(16).astype(np.float32), rng.standard_normal(7).astype(np.float32)]
    ref = O.fused_mlp_f64(x, ws, bs)
    assert O.max_rel_err(O.fused_mlp_f32(x, ws, bs), ref) < 1e-5
    assert np.all(ref >= 0)  # ReLU after the last layer too
    # identity weights and zero bias: relu(x)
    eye = np.eye(12, dtype=np.float32)
    assert np.array_equal(O.fused_mlp_f64(x, [eye], [np.zeros(12, np.float32)]), np.maximum(x, 0))
    # planted mistakes: W instead of W^T (non-square), and no ReLU on the last layer
    wrong = np.maximum(np.maximum(x @ ws[0].T + bs[0], 0) @ ws[1].T + bs[1], -np.inf)
    assert np.max(np.abs(wrong - ref)) > 1e-2
    w_sq = rng.standard_normal((12, 12)).astype(np.float32)
    assert np.max(np.abs(O.fused_mlp_f64(x, [w_sq], [bs[0][:12]]) - np.maximum(x @ w_sq + bs[0][:12], 0))) > 1e-2


def test_fused_mlp_validation_mirrors_reference():
    from barracuda_amd import fused_mlp
    dev = object()
    x = _t([4, 8], dev)
    w1, b1 = _t([16, 8], dev), _t([16], dev)
    with pytest.raises(InvalidInput, match=r"fused_mlp: weights len 1 != biases len 0"):
        fused_mlp(x, [w1], [])
    with pytest.raises(InvalidInput, match="at least one layer required"):
        fused_mlp(x, [], [])
    with pytest.raises(InvalidInput, match=r"fused_mlp: input must be 2D, got \[4, 8, 1\]"):
        fused_mlp(_t([4, 8, 1], dev), [w1], [b1])
    with pytest.raises(InvalidInput, match=r"fused_mlp: weight\[0\] must be 2D"):
        fused_mlp(x, [_t([16, 8, 1], dev)], [b1])
    with pytest.raises(InvalidInput, match=r"fused_mlp: weight\[1\] shape \[5, 7\] incompatible"):
        fused_mlp(x, [w1, _t([5, 7], dev)], [b1, _t([5], dev)])
    with pytest.raises(InvalidInput, match=r"fused_mlp: bias\[0\] shape mismatch"):
        fused_mlp(x, [w1], [_t([8], dev)])


# ------------------------------------------------------------------ f64 GEMM
def _gemm_cases():
    # ops/linalg/gemm_f64.rs tests: 2x2 basic, transpose A, transpose B, batched identities
    yield dict(a=[1, 2, 3, 4], b=[5, 6, 7, 8], mkn=(2, 2, 2), batch=1, ta=False, tb=False, want=[19, 22, 43, 50])
    yield dict(a=[1, 3, 2, 4], b=[5, 6, 7, 8], mkn=(2, 2, 2), batch=1, ta=True, tb=False, want=[19, 22, 43, 50])
    yield dict(a=[1, 2, 3, 4], b=[5, 7, 6, 8], mkn=(2, 2, 2), batch=1, ta=False, tb=True, want=[19, 22, 43, 50])
    b9 = list(range(1, 10))
    yield dict(a=[1, 0, 0, 0, 1, 0, 0, 0, 1, 2, 0, 0, 0, 2, 0, 0, 0, 2], b=b9 + b9, mkn=(3, 3, 3), batch=2,
               ta=False, tb=False, want=b9 + [2 * x for x in b9])


@pytest.mark.parametrize("case", list(_gemm_cases()), ids=["basic", "trans_a", "trans_b", "batched"])
def test_gemm_f64_oracle_reference_vectors(case):
    m, k, n = case["mkn"]
    got = O.gemm_f64_wgsl(case["a"], case["b"], m, k, n, case["batch"], trans_a=case["ta"], trans_b=case["tb"])
    assert got.tolist() == [float(x) for x in case["want"]]


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_f64_oracle_vs_longdouble_and_planted_transpose(ta, tb):
    rng = np.random.default_rng(13)
    batch, m, k, n = 2, 7, 19, 5
    a = rng.uniform(-1, 1, batch * m * k)
    b = rng.uniform(-1, 1, batch * k * n)
    got = O.gemm_f64_wgsl(a, b, m, k, n, batch, trans_a=ta, trans_b=tb)
    ref = O.gemm_longdouble(a, b, m, k, n, batch, ta, tb)
    assert np.max(np.abs(got - ref.astype(np.float64))) < 1e-14
    flipped = O.gemm_f64_wgsl(a, b, m, k, n, batch, trans_a=ta, trans_b=not tb)
    assert np.max(np.abs(flipped - got)) > 1e-3  # reading B with the wrong orientation is caught


def test_gemm_f64_oracle_alpha_beta():
    a, b = [1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]
    cin = np.array([1.0, -1.0, 0.5, 2.0])
    got = O.gemm_f64_wgsl(a, b, 2, 2, 2, 1, alpha=2.0, beta=3.0, c_in=cin)
    assert got.tolist() == [2 * 19 + 3 * 1.0, 2 * 22 - 3.0, 2 * 43 + 1.5, 2 * 50 + 6.0]
    nan_in = np.full(4, np.nan)
    assert O.gemm_f64_wgsl(a, b, 2, 2, 2, 1, alpha=1.0, beta=0.0, c_in=nan_in).tolist() == [19, 22, 43, 50]


def test_gemm_f64_validation_mirrors_reference():
    from barracuda_amd import GemmCachedF64, GemmF64
    with pytest.raises(InvalidInput, match="A: expected 4 elements, got 3"):
        GemmF64.execute(None, [1, 2, 3], [1, 2, 3, 4], 2, 2, 2, 1)
    with pytest.raises(InvalidInput, match="B: expected 8 elements, got 4"):
        GemmF64.execute_gemm_ex(None, [1] * 8, [1] * 4, 2, 2, 2, 2, 1.0, 0.0, True, False)
    with pytest.raises(InvalidInput, match=r"GemmCachedF64: B has 5 elements, expected batch×K×N=6"):
        GemmCachedF64(None, [1] * 5, 2, 3, 1)
