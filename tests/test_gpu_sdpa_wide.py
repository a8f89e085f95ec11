"""Attention at head dimensions above 128 on the MI355X vs the oracle.

The reference's attention ops accept any head_dim (ops/attention/mod.rs:
96-144, ops/flash_attention.rs:57-88, ops/grouped_query_attention/mod.rs:
84-147; a single-head MultiHeadAttention has head_dim = d_model,
ops/mha/mod.rs:152-187).  Here 129..256 run on the fused kernel's wider
instances and D > 256 on the chunked three-step path (GEMM, scaled and
masked row softmax, GEMM) in the context's workspace.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle;
the reference's f32 three-pass algorithm is held to the same bar where the
shapes are small enough for it.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from barracuda_amd import Attention, CausalAttention, FlashAttention, LcgStream, Tensor
from barracuda_amd import _native as N
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _up(dev, a):
    return Tensor.from_data(a, list(a.shape), dev)


def _sdpa(dev, q, k, v, causal):
    tq, tk, tv = _up(dev, q), _up(dev, k), _up(dev, v)
    return (tq.causal_attention(tk, tv) if causal else tq.attention(tk, tv)).to_numpy()


@pytest.mark.parametrize("B,H,Sq,Skv,D,causal", [
    (1, 2, 130, 130, 160, True), (2, 2, 128, 200, 160, False),
    (1, 2, 256, 256, 192, True), (1, 3, 100, 77, 192, False),
    (1, 2, 97, 97, 224, True),
    (1, 2, 256, 256, 256, True), (2, 2, 128, 128, 256, False), (1, 1, 130, 70, 256, False),
    (1, 2, 300, 300, 256, True), (1, 1, 1, 1, 256, False), (1, 1, 5, 9, 129, False),
    # D > 256: the chunked path
    (1, 2, 129, 129, 512, True), (1, 2, 64, 150, 512, False), (2, 1, 33, 33, 320, True),
    (1, 1, 40, 40, 1000, True), (1, 2, 257, 100, 260, False), (1, 1, 1, 1, 513, False),
    # causal chunks of 256 query rows over several heads, widths that take the
    # softmax with the scale and mask on its load (n % 4 == 0) and one that does not
    (1, 3, 600, 600, 320, True), (2, 2, 520, 520, 384, True), (1, 2, 514, 514, 300, True)])
def test_head_dims_vs_f64(dev, B, H, Sq, Skv, D, causal):
    _say(f"sdpa wide B={B} H={H} Sq={Sq} Skv={Skv} D={D} causal={causal}")
    rng = O.Lcg(B * 131 + H * 17 + Sq * 3 + Skv + D)
    q = rng.normal((B, H, Sq, D))
    k = rng.normal((B, H, Skv, D))
    v = rng.normal((B, H, Skv, D))
    got = _sdpa(dev, q, k, v, causal)
    assert O.max_rel_err(got, O.sdpa_f64(q, k, v, causal)) <= TOL
    if Sq == Skv:
        assert O.max_rel_err(got, O.attention_3pass_f32(q, k, v, causal)) <= TOL
    if causal:
        assert O.max_rel_err(got[:, :, 0, :], v[:, :, 0, :]) <= 1e-6  # row 0 attends to key 0 only


@pytest.mark.parametrize("D", [160, 256, 512])
def test_uniform_scores_give_the_mean_of_v(dev, D):
    """ops/attention/tests.rs:8-29 at a wide head: equal scores average V
    (causal row i: the mean of V[0..=i])."""
    _say(f"sdpa wide closed form D={D}")
    S = 70
    q = np.full((1, 1, S, D), 0.25, np.float32)
    k = np.full((1, 1, S, D), 0.5, np.float32)
    v = O.Lcg(D).normal((1, 1, S, D))
    got = _sdpa(dev, q, k, v, False)
    assert O.max_rel_err(got, np.broadcast_to(v.astype(np.float64).mean(axis=2, keepdims=True), got.shape)) <= 1e-5
    got = _sdpa(dev, q, k, v, True)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, S + 1)[None, None, :, None]
    assert O.max_rel_err(got, prefix) <= 1e-5


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 8, 2, 128, 256), (2, 4, 1, 100, 192), (1, 8, 2, 96, 512),
                                           (1, 6, 3, 64, 384)])
def test_gqa_vs_f64(dev, B, Hq, Hkv, S, D):
    _say(f"gqa wide B={B} Hq={Hq} Hkv={Hkv} S={S} D={D}")
    rng = O.Lcg(B * 7 + Hq * 5 + Hkv * 3 + S + D)
    q = rng.normal((B, Hq, S, D))
    k = rng.normal((B, Hkv, S, D))
    v = rng.normal((B, Hkv, S, D))
    got = _up(dev, q).grouped_query_attention(_up(dev, k), _up(dev, v)).to_numpy()
    assert O.max_rel_err(got, O.gqa_f64(q, k, v)) <= TOL
    assert O.max_rel_err(got, O.gqa_3pass_f32(q, k, v)) <= TOL


def _sdpa_ex(dev, B, H, Hkv, Sq, Skv, D, causal, q, ql, k, kl, v, vl, o, ol):
    lib = dev._lib
    with dev._lock:
        dev.check(lib.bch_sdpa_fwd_ex(dev.ctx, B, H, Hkv, Sq, Skv, D, float(np.float32(1) / np.sqrt(np.float32(D))),
                                      int(causal), C.c_void_p(q.ptr), N.AttnLayout(*ql), C.c_void_p(k.ptr),
                                      N.AttnLayout(*kl), C.c_void_p(v.ptr), N.AttnLayout(*vl), C.c_void_p(o.ptr),
                                      N.AttnLayout(*ol)), "sdpa_fwd_ex")


@pytest.mark.parametrize("B,H,Hkv,S,D,pad", [(2, 4, 2, 130, 256, 4), (1, 4, 2, 96, 192, 0), (2, 2, 1, 100, 512, 8),
                                              (1, 3, 3, 64, 300, 2)])
def test_causal_gqa_on_seq_major_padded_layouts(dev, B, H, Hkv, S, D, pad):
    """Q/O in [B, S, H, D] with a padded row (H*D + pad), K/V dense [B, Hkv, S, D]; causal."""
    _say(f"sdpa_ex wide causal B={B} H={H} Hkv={Hkv} S={S} D={D} pad={pad}")
    rng = O.Lcg(91 + S + D + pad)
    q = rng.normal((B, H, S, D))
    k = rng.normal((B, Hkv, S, D))
    v = rng.normal((B, Hkv, S, D))
    row = H * D + pad
    qs = np.zeros((B, S, row), np.float32)
    qs[:, :, :H * D] = q.transpose(0, 2, 1, 3).reshape(B, S, H * D)
    tq, tk, tv = _up(dev, qs), _up(dev, k), _up(dev, v)
    to = Tensor.from_data(np.full((B, S, row), 7.0, np.float32), [B, S, row], dev)
    lay = (S * row, D, row)
    _sdpa_ex(dev, B, H, Hkv, S, S, D, True, tq, lay, tk, (Hkv * S * D, S * D, D), tv, (Hkv * S * D, S * D, D),
             to, lay)
    out = to.to_numpy()
    assert np.all(out[:, :, H * D:] == 7.0)  # padding columns untouched
    got = out[:, :, :H * D].reshape(B, S, H, D).transpose(0, 2, 1, 3)
    assert O.max_rel_err(np.ascontiguousarray(got), O.gqa_f64(q, k, v, True)) <= TOL


@pytest.mark.parametrize("S,D", [(300, 256), (100, 512)])
def test_flash_attention_2d_wide(dev, S, D):
    """FlashAttention over [seq_len, head_dim] (ops/flash_attention.rs:57-88)."""
    _say(f"FlashAttention 2-D [{S}, {D}]")
    rng = O.Lcg(S + D)
    q, k, v = rng.normal((S, D)), rng.normal((S, D)), rng.normal((S, D))
    tq, tk, tv = (Tensor.from_data(t, [S, D], dev) for t in (q, k, v))
    got = FlashAttention(tq, tk, tv, 1).execute().to_numpy()
    ref = O.sdpa_f64(q[None, None], k[None, None], v[None, None], False)[0, 0]
    assert O.max_rel_err(got, ref) <= TOL


@pytest.mark.parametrize("B,Sq,Skv,D,H", [(2, 64, 64, 512, 1), (1, 40, 72, 512, 2), (2, 33, 33, 256, 1)])
def test_mha_wide_heads_vs_f64(dev, B, Sq, Skv, D, H):
    """MultiHeadAttention with head_dim = d_model / H above 128 (single head: d_model 512)."""
    _say(f"mha wide B={B} Sq={Sq} Skv={Skv} D={D} H={H}")
    rng = O.Lcg(B + Sq * 3 + Skv * 5 + D + H)
    q = rng.normal((B, Sq, D))
    k = rng.normal((B, Skv, D))
    v = rng.normal((B, Skv, D))
    ws = [rng.normal((D, D), 0.0, 1.0 / math.sqrt(D)) for _ in range(4)]
    out = _up(dev, q).multi_head_attention(_up(dev, k), _up(dev, v), *[_up(dev, w) for w in ws], H)
    assert out.shape() == [B, Sq, D]
    assert O.max_rel_err(out.to_numpy(), O.mha_f64(q, k, v, *ws, H)) <= TOL


@pytest.mark.parametrize("D", [256, 512])
def test_config_shape_wide(dev, D):
    """B=4, H=32, S=2048 (BASELINE config 5's shape) at head_dim 256 and 512,
    inputs N(0,1) from seed 4 generated in HBM (bch_fill_normal, bit-identical
    to the oracle's generator): three whole heads against f64, and every one
    of the 128 heads on a row sample touching each 128-query block."""
    B, H, S = 4, 32, 2048
    s = LcgStream(4, dev)
    tq, tk, tv = (s.normal([B, H, S, D]) for _ in range(3))
    q, k, v = tq.to_numpy(), tk.to_numpy(), tv.to_numpy()
    heads = [0, 77, 127]
    for causal in (False, True):
        _say(f"sdpa config shape D={D} causal={causal}")
        out = (CausalAttention(tq, tk, tv) if causal else Attention(tq, tk, tv)).execute().to_numpy()
        assert np.isfinite(out).all()
        got = out.reshape(B * H, S, D)[heads]
        ref = O.sdpa_f64(q, k, v, causal, heads=heads)
        err = O.max_rel_err(got, ref)
        _say(f"  max rel err vs f64 = {err:.3e}")
        assert err <= TOL
        rows = np.array([[blk * 128 + (h * 37 + blk * 11) % 128 for blk in range(16)] + [S - 1]
                         for h in range(B * H)], dtype=np.int32)
        refr = O.sdpa_f64_rows(q, k, v, causal, rows)
        gotr = np.take_along_axis(out.reshape(B * H, S, D), rows[:, :, None].astype(np.int64), axis=1)
        assert O.max_rel_err(gotr, refr) <= TOL
