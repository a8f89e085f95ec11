"""GELU, layer norm, the session's element-wise ops and the GELU GEMM
epilogue on the MI355X, through the C ABI, against the oracle.

Tolerance: max |x - ref| / max(|ref|, 1) <= 1e-4 against the f64 oracle (the
path's bar); GELU and layer norm are also held to the reference's own f32
restatements (gelu_wgsl_f32, layer_norm_f32) at the same bar.  add, sub,
mul, negate, scale and relu are single IEEE operations and are bit-exact
against numpy float32; fma is within 1 ulp of the exact a*b + c.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import GELU, Activation, LayerNorm, Tensor, TensorSession, nn
from barracuda_amd import _native as N
from barracuda_amd.error import InvalidInput, ShapeMismatch
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _ew(dev, op, a, b=None, c=None, scalar=0.0, offset=0):
    """bch_elementwise on device copies; `offset` elements shift every
    operand off 16-byte alignment (the scalar path)."""
    n = a.size
    bufs = []
    for x in (a, b, c):
        if x is None:
            bufs.append(None)
            continue
        t = Tensor.from_data(np.concatenate([np.zeros(offset, np.float32), x.reshape(-1)]), [n + offset], dev)
        bufs.append(t)
    out = Tensor.empty([n + offset], dev)
    p = lambda t: C.c_void_p(t.ptr + 4 * offset) if t is not None else None
    dev.check(dev._lib.bch_elementwise(dev.ctx, op, n, p(bufs[0]), p(bufs[1]), p(bufs[2]), float(scalar),
                                       p(out)), "elementwise")
    return out.to_vec()[offset:]


@pytest.mark.parametrize("n,offset", [(1, 0), (3, 0), (5, 1), (1000, 0), (1000003, 0), (4099, 3), (1 << 20, 2),
                                      ((1 << 23) + 5, 0)])
def test_gelu_vs_oracle(dev, n, offset):
    _say(f"gelu n={n} offset={offset}")
    x = O.Lcg(n + offset).normal((n,), 0.0, 4.0)
    x[: min(n, 4)] = np.array([0.0, 30.0, -30.0, 1e-3], np.float32)[: min(n, 4)]
    got = _ew(dev, N.BCH_EW_GELU, x, offset=offset)
    assert O.max_rel_err(got, O.gelu_f64(x)) <= 1e-5
    assert O.max_rel_err(got, O.gelu_wgsl_f32(x)) <= TOL
    if n >= 3:
        assert got[0] == 0.0 and got[1] == 30.0 and got[2] == 0.0


def test_gelu_extremes(dev):
    _say("gelu extremes")
    x = np.array([0.0, 1e-30, -1e-30, 5.0, -5.0, 88.0, -88.0, 1e30, -1e30, np.inf, -np.inf, np.nan], np.float32)
    got = _ew(dev, N.BCH_EW_GELU, x)
    ref = O.gelu_f64(x)
    fin = np.isfinite(ref)
    assert O.max_rel_err(got[fin], ref[fin]) <= 1e-6
    # +inf -> inf; -inf -> -0 (the formula is inf * 0 there: the oracle's NaN)
    assert got[9] == np.inf and got[10] == 0.0 and np.signbit(got[10]) and np.isnan(got[11])
    assert got[7] == np.float32(1e30) and got[8] == 0.0 and got[6] == 0.0


@pytest.mark.parametrize("offset,n", [(0, 300007), (1, 300007), (0, 6000001)])
def test_elementwise_ops_exact(dev, offset, n):
    """n = 6000001: every op moves at least 48 MB, the three-stream ones
    more than 64 MB (the non-temporal path)."""
    _say(f"elementwise ops offset={offset} n={n}")
    r = O.Lcg(9 + offset)
    a, b, c = r.normal((n,), 0.0, 3.0), r.normal((n,), 0.0, 3.0), r.normal((n,), 0.0, 3.0)
    assert np.array_equal(_ew(dev, N.BCH_EW_ADD, a, b, offset=offset), a + b)
    assert np.array_equal(_ew(dev, N.BCH_EW_SUB, a, b, offset=offset), a - b)
    assert np.array_equal(_ew(dev, N.BCH_EW_MUL, a, b, offset=offset), a * b)
    assert np.array_equal(_ew(dev, N.BCH_EW_NEG, a, offset=offset), -a)
    assert np.array_equal(_ew(dev, N.BCH_EW_SCALE, a, scalar=np.float32(0.37), offset=offset), a * np.float32(0.37))
    assert np.array_equal(_ew(dev, N.BCH_EW_RELU, a, offset=offset), np.maximum(a, np.float32(0.0)))
    got = _ew(dev, N.BCH_EW_FMA, a, b, c, offset=offset).astype(np.float64)
    exact = a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= ulp)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (7, 256), (9, 257), (4, 1000), (33, 2048), (8, 4096),
                                       (3, 4100), (2, 10000), (1, 65536),
                                       # one workgroup per row, the row in registers (4096 < cols <= 32768)
                                       (5, 4104), (300, 8192), (64, 32768), (2, 32772), (40, 40000), (3, 65536),
                                       (2, 65540),
                                       # other widths: scalar loads, the row in registers
                                       (65, 2047), (300, 4099), (70, 30001)])
def test_layer_norm_shapes(dev, rows, cols):
    _say(f"layer_norm rows={rows} cols={cols}")
    x = O.Lcg(rows * 7 + cols).normal((rows, cols), 1.5, 3.0)
    got = LayerNorm(Tensor.from_data(x, [rows, cols], dev), 1e-5).execute().to_numpy()
    _say(f"  kernel {dev._lib.bch_layer_norm_kernel_name(rows, cols, None, None).decode()}")
    assert O.max_rel_err(got, O.layer_norm_f64(x)) <= TOL
    assert O.max_rel_err(got, O.layer_norm_f32(x)) <= TOL


def test_layer_norm_reference_vectors_and_closed_forms(dev):
    """ops/layer_norm_wgsl.rs:166-192 (row means below 1e-5); [1,2,3,4]'s
    closed form; constant rows give exactly 0; in place; 3-D input."""
    _say("layer_norm reference vectors")
    y = Tensor.from_data(np.array([1, 2, 3, 4], np.float32), [1, 4], dev).layer_norm_wgsl(1e-5).to_numpy()
    assert abs(y.sum() / 4) < 1e-5
    want = (np.array([1, 2, 3, 4]) - 2.5) / np.sqrt(1.25 + 1e-5)
    assert np.max(np.abs(y[0] - want)) < 1e-6
    y2 = Tensor.from_data(np.arange(1, 7, dtype=np.float32), [2, 3], dev).layer_norm_wgsl(1e-5).to_numpy()
    assert np.all(np.abs(y2.mean(axis=1)) < 1e-5)
    z = Tensor.from_data(np.full((5, 2048), 3.0, np.float32), [5, 2048], dev).layer_norm_wgsl(1e-5).to_numpy()
    assert np.array_equal(z, np.zeros((5, 2048), np.float32))
    x = O.Lcg(3).normal((2, 16, 512))
    t = Tensor.from_data(x, [2, 16, 512], dev)
    dev.check(dev._lib.bch_layer_norm(dev.ctx, 32, 512, 1e-5, C.c_void_p(t.ptr), C.c_void_p(t.ptr)), "ln")
    assert O.max_rel_err(t.to_numpy(), O.layer_norm_f64(x)) <= TOL


def test_layer_norm_config_65536x2048(dev):
    """The softmax config's shape: [65536 x 2048], N(0, 3), seed 1."""
    _say("layer_norm 65536x2048 seed 1")
    x = O.Lcg(1).normal((65536, 2048), 0.0, 3.0)
    got = LayerNorm(Tensor.from_data(x, [65536, 2048], dev), 1e-5).execute().to_numpy()
    err = O.max_rel_err(got, O.layer_norm_f64(x))
    _say(f"  max rel err vs f64 = {err:.3e}")
    assert err <= TOL
    # every row has mean 0 and biased variance var / (var + eps)
    g = got.astype(np.float64)
    assert np.abs(g.mean(axis=1)).max() < 1e-5
    v = x.astype(np.float64).var(axis=1)
    assert np.abs(g.var(axis=1) - v / (v + 1e-5)).max() < 1e-4


def _gelu_ref(y):
    c = 0.7978845608
    return 0.5 * y * (1.0 + np.tanh(c * (y + 0.044715 * y ** 3)))


@pytest.mark.parametrize("m,n,k,transb", [(512, 384, 256, 1), (512, 384, 256, 0), (300, 200, 70, 1),
                                          (1, 11008, 4096, 1), (8, 11008, 4096, 1), (32, 11008, 4096, 1),
                                          (1, 4096, 1024, 0), (8, 4096, 1024, 0), (32, 4096, 1024, 0),
                                          (3, 1000, 300, 1)])
def test_linear_gelu_epilogue(dev, m, n, k, transb):
    _say(f"linear gelu m={m} n={n} k={k} transb={transb} kernel={dev._lib.bch_sgemm_kernel_name(m, n, k).decode()}")
    r = O.Lcg(m + n + k + transb)
    x = r.normal((m, k))
    w = r.normal((n, k) if transb else (k, n), 0.0, 0.05)
    bias = r.normal((n,), 0.0, 0.5)
    tx, tw, tb = (Tensor.from_data(a, list(a.shape), dev) for a in (x, w, bias))
    y = Tensor.empty([m, n], dev)
    dev.check(dev._lib.bch_sgemm_ex(dev.ctx, transb, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr),
                                    k if transb else n, C.c_void_p(tb.ptr), N.BCH_ACT_GELU, C.c_void_p(y.ptr), n),
              "linear")
    wd = w.astype(np.float64)
    pre = x.astype(np.float64) @ (wd.T if transb else wd) + bias.astype(np.float64)
    assert O.max_rel_err(y.to_numpy(), _gelu_ref(pre)) <= TOL


def test_nn_linear_and_fused_mlp_gelu(dev):
    _say("nn.linear / fused_mlp with GELU")
    r = O.Lcg(77)
    x = r.normal((64, 256))
    w1, b1 = r.normal((512, 256), 0.0, 0.05), r.normal((512,), 0.0, 0.1)
    w2, b2 = r.normal((128, 512), 0.0, 0.05), r.normal((128,), 0.0, 0.1)
    T = lambda a: Tensor.from_data(a, list(a.shape), dev)
    y = nn.linear(T(x), T(w1), T(b1), Activation.GELU).to_numpy()
    ref1 = _gelu_ref(x.astype(np.float64) @ w1.astype(np.float64).T + b1)
    assert O.max_rel_err(y, ref1) <= TOL
    z = nn.fused_mlp(T(x), [T(w1), T(w2)], [T(b1), T(b2)], Activation.GELU).to_numpy()
    ref2 = _gelu_ref(ref1 @ w2.astype(np.float64).T + b2)
    assert O.max_rel_err(z, ref2) <= TOL
    y0 = nn.linear(T(x), T(w1)).to_numpy()
    assert O.max_rel_err(y0, x.astype(np.float64) @ w1.astype(np.float64).T) <= TOL


def test_gelu_op_and_tensor_method(dev):
    _say("GELU op")
    x = O.Lcg(5).normal((33, 129), 0.0, 3.0)
    t = Tensor.from_data(x, [33, 129], dev)
    assert O.max_rel_err(GELU(t).execute().to_numpy(), O.gelu_f64(x)) <= TOL
    assert O.max_rel_err(t.gelu_wgsl().to_numpy(), O.gelu_f64(x)) <= TOL
    assert np.array_equal(t.relu().to_numpy(), np.maximum(x, np.float32(0)))


def test_session_elementwise_gelu_layer_norm_pipeline(dev):
    """A session pipeline over every new op (session/mod.rs:214-415), run in
    one batch, against numpy / the oracle."""
    _say("session pipeline: add sub mul negate fma scale relu gelu layer_norm reshape matmul")
    r = O.Lcg(101)
    a, b, c = r.normal((16, 64)), r.normal((16, 64)), r.normal((16, 64))
    w = r.normal((64, 32), 0.0, 0.2)
    s = TensorSession(dev)
    ta, tb, tc = s.tensor_with_shape(a, [16, 64]), s.tensor_with_shape(b, [16, 64]), s.tensor_with_shape(c, [16, 64])
    tw = s.tensor_with_shape(w, [64, 32])
    t_add, t_sub, t_mul = s.add(ta, tb), s.sub(ta, tb), s.mul(ta, tb)
    t_neg, t_fma, t_sc = s.negate(ta), s.fma(ta, tb, tc), s.scale(ta, 0.25)
    h = s.matmul(t_add, tw)
    t_relu, t_gelu = s.relu(h), s.gelu(h)
    t_ln = s.layer_norm(t_gelu, 32)
    t_flat = s.reshape(t_ln, [512])
    t_ln2 = s.layer_norm(t_flat, 64)
    assert s.num_ops() == 11
    s.run()
    assert np.array_equal(t_add.to_vec(), (a + b).reshape(-1))
    assert np.array_equal(t_sub.to_vec(), (a - b).reshape(-1))
    assert np.array_equal(t_mul.to_vec(), (a * b).reshape(-1))
    assert np.array_equal(t_neg.to_vec(), (-a).reshape(-1))
    assert np.array_equal(t_sc.to_vec(), (a * np.float32(0.25)).reshape(-1))
    exact = a.astype(np.float64) * b + c
    assert np.max(np.abs(t_fma.to_vec() - exact.reshape(-1)) / np.maximum(np.abs(exact.reshape(-1)), 1e-30)) < 1.2e-7
    hv = ((a + b).astype(np.float64) @ w.astype(np.float64))
    assert O.max_rel_err(t_relu.to_vec(), np.maximum(hv, 0.0).reshape(-1)) <= TOL
    g = _gelu_ref(hv)
    assert O.max_rel_err(t_gelu.to_vec(), g.reshape(-1)) <= TOL
    ln = (g - g.mean(axis=1, keepdims=True)) / np.sqrt(g.var(axis=1, keepdims=True) + 1e-5)
    assert O.max_rel_err(t_ln.to_vec(), ln.reshape(-1)) <= TOL
    assert t_flat.shape() == [512] and t_flat.buffer_id == t_ln.buffer_id
    ln2 = ln.reshape(8, 64)
    ln2 = (ln2 - ln2.mean(axis=1, keepdims=True)) / np.sqrt(ln2.var(axis=1, keepdims=True) + 1e-5)
    assert O.max_rel_err(t_ln2.to_vec(), ln2.reshape(-1)) <= TOL


def test_session_new_op_errors(dev):
    _say("session op errors")
    s = TensorSession(dev)
    x = s.tensor_with_shape(np.ones(12, np.float32), [3, 4])
    y = s.tensor_with_shape(np.ones(12, np.float32), [4, 3])
    with pytest.raises(ShapeMismatch):
        s.add(x, y)
    with pytest.raises(ShapeMismatch):
        s.fma(x, x, y)
    with pytest.raises(InvalidInput, match="layer_norm: total 12 not divisible by feature_size 5"):
        s.layer_norm(x, 5)
    with pytest.raises(ShapeMismatch):
        s.reshape(x, [5, 2])
    assert s.num_ops() == 0


def _rows_offset(dev, fn, x, offset_in, offset_out):
    """Run fn(ctx, rows, cols, pin, pout) on buffers whose data starts offset_* floats into a larger
    allocation (so the pointers are 4-byte but not 16-byte aligned when the offset is odd)."""
    rows, cols = x.shape
    n = rows * cols
    tin = Tensor.from_data(np.concatenate([np.zeros(offset_in, np.float32), x.reshape(-1)]), [n + offset_in], dev)
    tout = Tensor.from_data(np.full(n + offset_out + 3, 7.0, np.float32), [n + offset_out + 3], dev)
    pin, pout = C.c_void_p(tin.ptr + 4 * offset_in), C.c_void_p(tout.ptr + 4 * offset_out)
    with dev._lock:
        dev.check(fn(dev.ctx, rows, cols, pin, pout), "row op")
    out = tout.to_numpy()
    assert np.all(out[:offset_out] == 7.0) and np.all(out[offset_out + n:] == 7.0)  # nothing written outside
    return out[offset_out:offset_out + n].reshape(rows, cols), pin, pout


@pytest.mark.parametrize("rows,cols", [(300, 2048), (40, 8192), (6, 32768)])
@pytest.mark.parametrize("oin,oout", [(1, 1), (1, 0), (0, 1)])
def test_layer_norm_unaligned_buffers(dev, rows, cols, oin, oout):
    """Widths divisible by 4 on buffers one float off 16-byte alignment take the scalar
    register kernels; the reported kernel name follows the same choice."""
    x = O.Lcg(rows + cols + oin).normal((rows, cols), 1.5, 3.0)
    lib = dev._lib
    got, pin, pout = _rows_offset(dev, lambda c, r, k, a, b: lib.bch_layer_norm(c, r, k, 1e-5, a, b), x, oin, oout)
    name = lib.bch_layer_norm_kernel_name(rows, cols, pin, pout).decode()
    _say(f"layer_norm unaligned rows={rows} cols={cols} in+{oin} out+{oout}: {name}")
    assert name.startswith("layer_norm_wgs")
    assert O.max_rel_err(got, O.layer_norm_f64(x)) <= TOL


def test_layer_norm_row_count_past_one_grid(dev):
    """2^26 + 3 rows of 4: the wavefront-per-row kernel in one grid would need more than 2^32
    threads; the call runs in launches of 2^21 rows.  Rows at every launch boundary and a sample
    against f64; every row's mean is ~0."""
    rows, cols = (1 << 26) + 3, 4
    _say(f"layer_norm rows={rows} cols={cols}")
    from barracuda_amd import LcgStream
    x = LcgStream(44, dev).normal([rows, cols], 0.5, 2.0)
    y = Tensor.empty([rows, cols], dev)
    with dev._lock:
        dev.check(dev._lib.bch_layer_norm(dev.ctx, rows, cols, 1e-5, C.c_void_p(x.ptr), C.c_void_p(y.ptr)), "ln")
    xs, ys = x.to_numpy().reshape(rows, cols), y.to_numpy().reshape(rows, cols)
    # every row's mean is ~0 (rows whose variance is near eps amplify the f32 rounding of x - mean)
    assert np.max(np.abs(ys.astype(np.float64).mean(axis=1))) < 1e-4
    edge = [b + d for b in range(0, rows + 1, 1 << 21) for d in (-1, 0, 1)]
    sample = sorted({r for r in edge if 0 <= r < rows} | set(range(0, rows, 99991)) | {rows - 1})
    assert O.max_rel_err(ys[sample], O.layer_norm_f64(np.ascontiguousarray(xs[sample]))) <= TOL
