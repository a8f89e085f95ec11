"""Grouped-query and multi-head attention on the MI355X (bch_sdpa_fwd_ex) vs
the oracle.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle
(oracle.gqa_f64, oracle.mha_f64); the reference's f32 three-pass GQA
algorithm is held to the same bar on the same inputs.
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


def _say(msg):
    print(msg, flush=True)


def _up(dev, a):
    return Tensor.from_data(a, list(a.shape), dev)


def test_gqa_reference_vector(dev):
    # ops/grouped_query_attention/tests.rs:21-38
    _say("gqa reference vector [1,8,4,4] / [1,2,4,4]")
    q = np.full((1, 8, 4, 4), 0.5, np.float32)
    kv = np.full((1, 2, 4, 4), 0.5, np.float32)
    out = _up(dev, q).grouped_query_attention(_up(dev, kv), _up(dev, kv))
    assert out.shape() == [1, 8, 4, 4]
    assert np.max(np.abs(out.to_numpy() - 0.5)) <= 1e-6


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [
    (1, 4, 4, 64, 32),      # group 1 = plain attention
    (2, 8, 2, 256, 64),     # group 4, full tiles
    (1, 8, 1, 128, 128),    # multi-query attention
    (2, 6, 3, 100, 48),     # ragged rows and head dim
    (1, 32, 8, 512, 128),   # LLaMA-style head ratio
])
def test_gqa_vs_f64(dev, B, Hq, Hkv, S, D):
    _say(f"gqa B={B} Hq={Hq} Hkv={Hkv} S={S} D={D}")
    rng = O.Lcg(B * 7 + Hq * 5 + Hkv * 3 + S + D)
    q = rng.normal((B, Hq, S, D))
    k = rng.normal((B, Hkv, S, D))
    v = rng.normal((B, Hkv, S, D))
    got = _up(dev, q).grouped_query_attention(_up(dev, k), _up(dev, v)).to_numpy()
    assert O.max_rel_err(got, O.gqa_f64(q, k, v)) <= TOL
    if S <= 256:
        assert O.max_rel_err(got, O.gqa_3pass_f32(q, k, v)) <= TOL


def _sdpa_ex(dev, B, H, Hkv, Sq, Skv, D, causal, q, ql, k, kl, v, vl, o, ol):
    lib = dev._lib
    with dev._lock:
        dev.check(lib.bch_sdpa_fwd_ex(dev.ctx, B, H, Hkv, Sq, Skv, D, float(np.float32(1) / np.sqrt(np.float32(D))),
                                      int(causal), C.c_void_p(q.ptr), N.AttnLayout(*ql), C.c_void_p(k.ptr),
                                      N.AttnLayout(*kl), C.c_void_p(v.ptr), N.AttnLayout(*vl), C.c_void_p(o.ptr),
                                      N.AttnLayout(*ol)), "sdpa_fwd_ex")


@pytest.mark.parametrize("B,H,Hkv,S,D,pad", [(2, 4, 2, 128, 64, 0), (1, 4, 4, 96, 40, 4), (2, 8, 2, 160, 128, 8)])
def test_causal_gqa_on_seq_major_padded_layouts(dev, B, H, Hkv, S, D, pad):
    """Q/O in [B, S, H, D] with a padded row (H*D + pad), K/V dense [B, Hkv, S, D]; causal."""
    _say(f"sdpa_ex causal B={B} H={H} Hkv={Hkv} S={S} D={D} pad={pad}")
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


@pytest.mark.parametrize("sq,skv", [(8, 8), (8, 16)])
def test_mha_reference_vectors(dev, sq, skv):
    # ops/mha/tests.rs:9-56 and :98-149: closed form 0.4096 everywhere
    _say(f"mha reference vector sq={sq} skv={skv}")
    q = _up(dev, np.full((2, sq, 64), 0.5, np.float32))
    k = _up(dev, np.full((2, skv, 64), 0.5, np.float32))
    v = _up(dev, np.full((2, skv, 64), 1.0, np.float32))
    w = _up(dev, np.full((64, 64), 0.01, np.float32))
    out = q.multi_head_attention(k, v, w, w, w, w, 8)
    assert out.shape() == [2, sq, 64]
    want = O.mha_f64(np.full((2, sq, 64), 0.5, np.float32), np.full((2, skv, 64), 0.5, np.float32),
                     np.full((2, skv, 64), 1.0, np.float32), *(np.full((64, 64), 0.01, np.float32),) * 4, 8)
    assert O.max_rel_err(out.to_numpy(), want) <= 1e-5


@pytest.mark.parametrize("B,Sq,Skv,D,H", [(2, 64, 64, 256, 4), (2, 37, 96, 256, 8), (1, 128, 128, 512, 4),
                                           (3, 16, 16, 96, 3)])
def test_mha_vs_f64(dev, B, Sq, Skv, D, H):
    _say(f"mha B={B} Sq={Sq} Skv={Skv} D={D} H={H}")
    rng = O.Lcg(B + Sq * 3 + Skv * 5 + D + H)
    q = rng.normal((B, Sq, D))
    k = rng.normal((B, Skv, D))
    v = rng.normal((B, Skv, D))
    ws = [rng.normal((D, D), 0.0, 1.0 / math.sqrt(D)) for _ in range(4)]
    out = _up(dev, q).multi_head_attention(_up(dev, k), _up(dev, v), *[_up(dev, w) for w in ws], H)
    assert out.shape() == [B, Sq, D]
    assert O.max_rel_err(out.to_numpy(), O.mha_f64(q, k, v, *ws, H)) <= TOL
