"""Fused attention forward on the MI355X vs the oracle (bch_sdpa_fwd).

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle;
the reference's own f32 algorithms (three-pass K6/K7/K9 and the CPU causal
path) are held to the same bar on the same inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from barracuda_amd import Attention, CausalAttention, FlashAttention, Tensor
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _sdpa(dev, q, k, v, causal):
    tq = Tensor.from_data(q, list(q.shape), dev)
    tk = Tensor.from_data(k, list(k.shape), dev)
    tv = Tensor.from_data(v, list(v.shape), dev)
    if causal:
        return tq.causal_attention(tk, tv).to_numpy()
    return tq.attention(tk, tv).to_numpy()


def test_closed_forms(dev, golden):
    for case in golden["attention"]:
        _say(f"attention golden {case['name']}")
        sq = case.get("shape_q", case.get("shape"))
        skv = case.get("shape_kv", case.get("shape"))
        q = np.array(case["q"], dtype=np.float32).reshape(sq)
        k = np.array(case["k"], dtype=np.float32).reshape(skv)
        v = np.array(case["v"], dtype=np.float32).reshape(skv)
        got = _sdpa(dev, q, k, v, case["causal"]).reshape(-1)
        assert np.max(np.abs(got - np.array(case["expected"]))) <= max(case["tol"], 1e-5), case["name"]


@pytest.mark.parametrize("B,H,Sq,Skv,D,causal", [
    (1, 1, 1, 1, 1, False), (1, 1, 5, 5, 3, True), (2, 3, 7, 7, 8, False), (1, 2, 4, 9, 16, False),
    (1, 1, 33, 33, 32, True), (2, 2, 100, 100, 64, True), (1, 2, 128, 128, 128, False),
    (1, 2, 256, 256, 128, True), (1, 1, 130, 70, 128, False), (1, 1, 64, 300, 100, False),
    (2, 1, 257, 257, 128, True),
    # grids that are a multiple of 8 take the XCD-contiguous head-major order (non-causal)
    (2, 4, 256, 256, 64, False), (1, 8, 384, 384, 32, False), (1, 8, 384, 320, 128, False)])
def test_shapes_vs_f64(dev, B, H, Sq, Skv, D, causal):
    _say(f"sdpa B={B} H={H} Sq={Sq} Skv={Skv} D={D} causal={causal}")
    rng = O.Lcg(B * 131 + H * 17 + Sq * 3 + Skv + D)
    q = rng.normal((B, H, Sq, D))
    k = rng.normal((B, H, Skv, D))
    v = rng.normal((B, H, Skv, D))
    got = _sdpa(dev, q, k, v, causal)
    ref = O.sdpa_f64(q, k, v, causal)
    err = O.max_rel_err(got, ref)
    assert err <= TOL
    if Sq == Skv:
        ref32 = O.attention_3pass_f32(q, k, v, causal)
        assert O.max_rel_err(got, ref32) <= TOL
    if causal:
        assert O.max_rel_err(got[:, :, 0, :], v[:, :, 0, :]) <= 1e-6  # row 0 attends to key 0 only


def test_flash_attention_2d(dev):
    _say("FlashAttention 2-D [200, 64]")
    rng = O.Lcg(21)
    q, k, v = rng.normal((200, 64)), rng.normal((200, 64)), rng.normal((200, 64))
    tq, tk, tv = (Tensor.from_data(t, [200, 64], dev) for t in (q, k, v))
    got = FlashAttention(tq, tk, tv, 1).execute().to_numpy()
    ref = O.sdpa_f64(q[None, None], k[None, None], v[None, None], False)[0, 0]
    assert O.max_rel_err(got, ref) <= TOL


def test_config_b4_h32_s2048_d128(dev):
    """B=4, H=32, S=2048, D=128, N(0,1), seed 4, scale 1/sqrt(128);
    causal and non-causal; f64 oracle and the reference f32 algorithms on sampled heads."""
    _say("sdpa config B=4 H=32 S=2048 D=128 seed 4")
    rng = O.Lcg(4)
    shape = (4, 32, 2048, 128)
    q, k, v = rng.normal(shape), rng.normal(shape), rng.normal(shape)
    tq, tk, tv = (Tensor.from_data(t, list(shape), dev) for t in (q, k, v))
    heads = [0, 37, 127]
    for causal in (False, True):
        _say(f"  causal={causal}")
        out = (CausalAttention(tq, tk, tv) if causal else Attention(tq, tk, tv)).execute().to_numpy()
        got = out.reshape(128, 2048, 128)[heads]
        ref = O.sdpa_f64(q, k, v, causal, heads=heads)
        err = O.max_rel_err(got, ref)
        _say(f"  max rel err vs f64 = {err:.3e}")
        assert err <= TOL
        ref32 = O.attention_3pass_f32(q, k, v, causal, heads=[37])
        assert O.max_rel_err(got[1], ref32[0]) <= TOL
        assert np.isfinite(out).all()
        # every one of the 128 heads on a row sample that touches each of its
        # 16 query blocks of 128 (the row inside the block moves with the
        # head and the block) and the last row: a head or block mapping slip
        # anywhere in the grid fails here
        rows = np.array([[blk * 128 + (h * 37 + blk * 11) % 128 for blk in range(16)] + [2047]
                         for h in range(128)], dtype=np.int32)
        refr = O.sdpa_f64_rows(q, k, v, causal, rows)
        gotr = np.take_along_axis(out.reshape(128, 2048, 128), rows[:, :, None].astype(np.int64), axis=1)
        err_all = O.max_rel_err(gotr, refr)
        _say(f"  all 128 heads x 17 rows: max rel err vs f64 = {err_all:.3e}")
        assert err_all <= TOL
