"""bch_softmax_rows_f64 (the row softmax of ml.attention, ml/forward.rs:
130-140) and the f64 attention built on it, on the MI355X through the C ABI,
against the oracle's restatement of the handler's loops.

Tolerance: |x - ref| <= 1e-13 |ref| + 1e-300 elementwise (f64 against f64:
exp differs by at most an ulp or two between the device's and the host's
libm, and the row sum is added in a different order).  Non-finite values
must match exactly (NaN where the reference's row is NaN).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import F64Buffer, linalg
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _run(dev, x, offset=0, inplace=False):
    """x [rows, cols] through bch_softmax_rows_f64; `offset` doubles shift
    both buffers off 16-byte alignment."""
    rows, cols = x.shape
    n = x.size
    src = F64Buffer(dev, n + offset).upload(np.concatenate([np.zeros(offset), x.reshape(-1)]))
    dst = src if inplace else F64Buffer(dev, n + offset)
    pin, pout = src.ptr + 8 * offset, dst.ptr + 8 * offset
    name = dev._lib.bch_softmax_rows_f64_kernel_name(rows, cols, C.c_void_p(pin), C.c_void_p(pout)).decode()
    with dev._lock:
        dev.check(dev._lib.bch_softmax_rows_f64(dev.ctx, rows, cols, C.c_void_p(pin), C.c_void_p(pout)),
                  "softmax_f64")
    return dst.to_vec()[offset:].reshape(rows, cols), name


def _close(got, want):
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
    err = np.abs(got[fin] - want[fin]) - (1e-13 * np.abs(want[fin]) + 1e-300)
    assert err.size == 0 or np.max(err) <= 0.0, float(np.max(err))


@pytest.mark.parametrize("rows,cols,offset,kernel", [
    (1, 1, 0, "softmax_f64_rows<1,1,1>"), (3, 2, 0, "softmax_f64_rows<1,2,1>"),
    (7, 64, 0, "softmax_f64_rows<1,2,1>"), (5, 65, 0, "softmax_f64_rows<2,1,1>"),
    (9, 300, 0, "softmax_f64_rows<4,2,1>"), (4, 512, 1, "softmax_f64_rows<8,1,1>"),
    (3, 513, 0, "softmax_f64_rows<4,1,4>"), (6, 2048, 0, "softmax_f64_rows<4,2,4>"),
    (5, 2047, 0, "softmax_f64_rows<8,1,4>"), (7, 1030, 0, "softmax_f64_rows<4,2,4>"),
    (2, 2049, 0, "softmax_f64_rows<16,1,4>"), (3, 100003, 0, "softmax_f64_block"),
    (3, 4096, 0, "softmax_f64_rows<8,2,4>"), (2, 8192, 0, "softmax_f64_rows<16,2,4>"),
    (2, 8191, 0, "softmax_f64_rows<32,1,4>"), (3, 6000, 1, "softmax_f64_rows<32,1,4>"),
    (2, 8194, 0, "softmax_f64_block"),
    (4099, 128, 0, "softmax_f64_rows<1,2,1>"), (1025, 1000, 1, "softmax_f64_rows<4,1,4>"),
    (4097, 700, 0, "softmax_f64_rows<2,2,4>")])
def test_softmax_f64_shapes_vs_oracle(dev, rows, cols, offset, kernel):
    _say(f"softmax_f64 rows={rows} cols={cols} offset={offset}")
    x = O.Lcg(rows * 7919 + cols).normal((rows, cols)).astype(np.float64) * 20.0
    got, name = _run(dev, x, offset)
    assert name == kernel
    _close(got, O.ml_softmax_rows_f64(x))
    assert np.all(np.abs(got.sum(axis=1) - 1.0) < 1e-13)


def test_softmax_f64_in_place_and_special_rows(dev):
    _say("softmax_f64 in place, NaN / inf / huge rows")
    x = O.Lcg(5).normal((6, 40)).astype(np.float64)
    x[1, 7] = np.nan                 # f64::max skips it, exp(NaN - m) poisons the row
    x[2, :] = np.inf * np.sign(x[2, :])  # +inf entries: inf - inf -> NaN row
    x[3, :] = -np.inf                # max -inf: every exp(-inf + inf) is NaN
    x[4, :] = 1e300 * np.sign(x[4, :])
    x[5, :] = 2.0                    # equal row: exactly 1/40 after the division
    for inplace in (False, True):
        got, _ = _run(dev, x, inplace=inplace)
        want = O.ml_softmax_rows_f64(x)
        _close(got, want)
        assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2])) and np.all(np.isnan(got[3]))
        assert np.array_equal(got[5], np.full(40, 1.0 / 40.0))
    big = np.tile(np.array([[1000.0, 1001.0, 999.0, -1e308]]), (5, 300))
    for inplace in (False, True):
        got, name = _run(dev, big, inplace=inplace)
        assert name == "softmax_f64_rows<4,2,4>"
        _close(got, O.ml_softmax_rows_f64(big))


def test_softmax_rows_f64_host_helper(dev):
    _say("linalg.softmax_rows_f64")
    x = O.Lcg(9).normal((2, 3, 50)).astype(np.float64)
    _close(linalg.softmax_rows_f64(dev, x).reshape(6, 50), O.ml_softmax_rows_f64(x.reshape(6, 50)))


@pytest.mark.parametrize("sq,sk,dk,dv", [(1, 1, 1, 1), (16, 16, 8, 8), (100, 257, 64, 33), (512, 512, 128, 128),
                                         (7, 3000, 16, 5)])
def test_attention_f64_vs_oracle(dev, sq, sk, dk, dv):
    """linalg.attention_f64 (bch_dgemm, bch_softmax_rows_f64, bch_dgemm) against
    ml/forward.rs:121-150 restated: max |x - ref| / max(|ref|, 1) <= 1e-12."""
    _say(f"attention_f64 sq={sq} sk={sk} dk={dk} dv={dv}")
    rng = O.Lcg(sq + 3 * sk + 5 * dk + 7 * dv)
    q, k, v = (rng.normal(s).astype(np.float64) for s in ((sq, dk), (sk, dk), (sk, dv)))
    got = linalg.attention_f64(dev, q, k, v)
    want = O.ml_attention_f64(q, k, v)
    assert np.max(np.abs(got - want)) <= 1e-12 * max(1.0, np.max(np.abs(want)))


def test_softmax_f64_row_count_past_one_grid(dev):
    """2^26 + 3 rows of 2 doubles: one grid of the wavefront-per-row kernel would need more than
    2^32 threads; the call runs in launches of 2^21 rows.  Rows at every launch boundary and a
    sample against the handler's loop restated."""
    rows, cols = (1 << 26) + 3, 2
    _say(f"softmax_f64 rows={rows} cols={cols}")
    rng = np.random.default_rng(46)
    x = rng.normal(0.0, 3.0, (rows, cols))
    got, name = _run(dev, x)
    _say(f"  kernel {name}")
    edge = [b + d for b in range(0, rows + 1, 1 << 21) for d in (-1, 0, 1)]
    sample = sorted({r for r in edge if 0 <= r < rows} | set(range(0, rows, 99991)) | {rows - 1})
    _close(got[sample], O.ml_softmax_rows_f64(np.ascontiguousarray(x[sample])))
    assert np.max(np.abs(got.sum(axis=1) - 1.0)) < 1e-12
