"""The tensor wire paths' JSON-RPC handlers (barracuda_amd/ipc.py) with the
reference's method vectors: ipc/methods_tests/batch_tests.rs,
ipc/methods_tests/tensor_fhe_tests.rs, ipc/methods_coverage_tests/
sprint56b_tests.rs:618-669 and the wire contract in ipc/methods/batch.rs:
8-37.  The CPU tests cover routing and every validation path (no device);
the GPU tests run the handlers through the HIP path."""
from __future__ import annotations

import numpy as np
import pytest

from barracuda_amd import ipc
from oracle import bc_oracle as O

TOL = 1e-4


@pytest.fixture
def headless():
    return ipc.TensorPrimal(None)


def _err(resp):
    assert "error" in resp and "result" not in resp, resp
    return resp["error"]


# ---- CPU: routing and validation ------------------------------------------------
def test_normalize_and_unknown_method(headless):
    assert ipc.normalize_method("barracuda.tensor.matmul") == "tensor.matmul"
    assert ipc.normalize_method("tensor.matmul") == "tensor.matmul"
    e = _err(ipc.dispatch(headless, "tensor.quantum", {}, 9))
    assert e["code"] == ipc.METHOD_NOT_FOUND and e["message"] == "Unknown method: tensor.quantum"
    r = ipc.dispatch(headless, "barracuda.tensor.batch.submit", {}, 10)
    assert r["id"] == 10 and r["jsonrpc"] == "2.0" and _err(r)["code"] == ipc.INVALID_PARAMS


def test_batch_error_vectors(headless):
    """ipc/methods_tests/batch_tests.rs, each case's params and expected code."""
    sub = lambda params, i: ipc.tensor_batch_submit(headless, params, i)
    assert _err(sub({}, 1))["code"] == ipc.INVALID_PARAMS                       # missing ops
    assert _err(sub({"ops": []}, 2))["code"] == ipc.INVALID_PARAMS              # empty ops
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [4], "data": [1, 2, 3, 4]}]}, 3))
    assert e["code"] == ipc.INTERNAL_ERROR                                         # no GPU
    e = _err(sub({"ops": [{"op": "quantum_entangle", "alias": "x"}]}, 4))
    assert e["code"] == ipc.INVALID_PARAMS and "quantum_entangle" in e["message"]
    e = _err(sub({"ops": [{"op": "relu", "alias": "y", "input": "nonexistent"}]}, 5))
    assert e["code"] == ipc.INVALID_PARAMS and "nonexistent" in e["message"]
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [2, 3], "data": [1.0]}]}, 6))
    assert e["code"] == ipc.INVALID_PARAMS and "data length" in e["message"]
    e = _err(sub({"ops": [{"op": "readback", "alias": "out", "input": "missing"}]}, 7))
    assert e["code"] == ipc.INVALID_PARAMS and "missing" in e["message"]
    assert _err(sub({"ops": [{"op": "readback", "alias": "out"}]}, 8))["code"] == ipc.INVALID_PARAMS
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [4]}, {"op": "layer_norm", "alias": "y"}]}, 9))
    assert e["code"] == ipc.INVALID_PARAMS and "requires 'input'" in e["message"]
    e = _err(sub({"ops": [{"op": "gelu", "alias": "y", "input": "ghost"}]}, 10))
    assert e["code"] == ipc.INVALID_PARAMS and "ghost" in e["message"]
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [4]},
                          {"op": "layer_norm", "alias": "y", "input": "x"}]}, 11))
    assert e["code"] == ipc.INVALID_PARAMS and "feature_size" in e["message"]
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [4]},
                          {"op": "scale", "alias": "y", "input": "x"}]}, 12))
    assert e["message"] == "ops[1]: scale requires 'scalar'"
    e = _err(sub({"ops": [{"op": "create", "alias": "x", "shape": [4]},
                          {"op": "fma", "alias": "y", "a": "x", "b": "x"}]}, 13))
    assert e["message"] == "ops[1]: fma requires 'c' alias"
    e = _err(sub({"ops": [{"alias": "x"}]}, 14))
    assert e["message"] == "ops[0]: missing 'op' field"


def test_tensor_matmul_error_vectors(headless):
    """tensor_fhe_tests.rs: unknown ids, missing lhs_id / rhs_id."""
    e = _err(ipc.tensor_matmul(headless, {"lhs_id": "a", "rhs_id": "b"}, 15))
    assert e["code"] == ipc.INVALID_PARAMS and "Tensor not found" in e["message"]
    assert _err(ipc.tensor_matmul(headless, {"rhs_id": "b"}, 160))["message"] == "Missing required param: lhs_id"
    assert _err(ipc.tensor_matmul(headless, {"lhs_id": "a"}, 161))["message"] == "Missing required param: rhs_id"
    assert _err(ipc.tensor_create(headless, {}, 14))["code"] == ipc.INVALID_PARAMS
    e = _err(ipc.tensor_create(headless, {"shape": [2, 3], "data": [1.0]}, 16))
    assert e["message"] == "data length 1 does not match shape product 6"
    e = _err(ipc.tensor_create(headless, {"shape": [2, 3]}, 13))
    assert e["code"] == ipc.INTERNAL_ERROR and e["message"] == "No GPU device available"


def test_inline_handler_error_vectors(headless):
    """ml_tests.rs:84-126 and sprint56b_tests.rs:585-615, plus every other
    validation answer of ml/forward.rs:83-117 and tensor.rs:496-537; a valid
    request without a device is INTERNAL_ERROR."""
    att = lambda params, i: ipc.dispatch(headless, "ml.attention", params, i)
    for i, (params, msg) in enumerate((
            ({"k": [[1.0]], "v": [[1.0]]}, "Missing required param: q (2D array)"),
            ({"q": [[1.0]], "v": [[1.0]]}, "Missing required param: k (2D array)"),
            ({"q": [[1.0]], "k": [[1.0]]}, "Missing required param: v (2D array)"),
            ({"q": [], "k": [[1.0]], "v": [[1.0]]}, "q, k, v must be non-empty"),
            ({"q": [[]], "k": [[1.0]], "v": [[1.0]]}, "Key dimension must be > 0"),
            ({"q": [[1.0, 2.0]], "k": [[1.0]], "v": [[1.0]]}, "q and k must have matching inner dimension"),
            ({"q": [[1.0], [1.0, 2.0]], "k": [[1.0]], "v": [[1.0]]}, "q and k must have matching inner dimension"),
            ({"q": [[1.0]], "k": [[1.0], [2.0]], "v": [[1.0]]},
             "v must have same sequence length as k with consistent column count"),
            ({"q": [[1.0]], "k": [[1.0], [2.0]], "v": [[1.0], [1.0, 2.0]]},
             "v must have same sequence length as k with consistent column count"),
            ({"q": "x", "k": [[1.0]], "v": [[1.0]]}, "Missing required param: q (2D array)"))):
        e = _err(att(params, 310 + i))
        assert e["code"] == ipc.INVALID_PARAMS and e["message"] == msg, (params, e)
    # params.rs:21-30: rows that are not arrays and entries that are not numbers are dropped
    e = _err(att({"q": [[1.0, "a", True, 2.0], "row"], "k": [[1.0, 2.0]], "v": [[3.0]]}, 330))
    assert e["code"] == ipc.INTERNAL_ERROR and e["message"] == "No GPU device available"
    mm = lambda params, i: ipc.dispatch(headless, "barracuda.tensor.matmul_inline", params, i)
    for i, (params, msg) in enumerate((
            ({}, "Missing required params: lhs and rhs (2D arrays)"),
            ({"lhs": [[1.0]]}, "Missing required params: lhs and rhs (2D arrays)"),
            ({"lhs": [], "rhs": [[1.0]]}, "lhs must be non-empty"),
            ({"lhs": [[]], "rhs": [[1.0]]}, "lhs rows must have consistent length"),
            ({"lhs": [[1.0], [1.0, 2.0]], "rhs": [[1.0]]}, "lhs rows must have consistent length"),
            ({"lhs": [[1.0]], "rhs": []}, "rhs must be non-empty"),
            ({"lhs": [[1.0, 2.0]], "rhs": [[1.0], [2.0], [3.0]]}, "Shape mismatch: lhs is [1x2], rhs must be [2x1]"),
            ({"lhs": [[1.0, 2.0]], "rhs": [[1.0, 2.0], [3.0]]}, "Shape mismatch: lhs is [1x2], rhs must be [2x2]"))):
        e = _err(mm(params, 200 + i))
        assert e["code"] == ipc.INVALID_PARAMS and e["message"] == msg, (params, e)
    e = _err(mm({"lhs": [[1.0, 2.0]], "rhs": [[1.0], [2.0]]}, 220))
    assert e["code"] == ipc.INTERNAL_ERROR and e["message"] == "No GPU device available"


# ---- GPU: the handlers on the HIP path ----------------------------------------------
@pytest.fixture
def primal(dev):
    return ipc.TensorPrimal(dev)


def _create(primal, shape, data, i):
    r = ipc.dispatch(primal, "tensor.create", {"shape": shape, "data": data}, i)
    assert "result" in r, r
    assert r["result"]["shape"] == shape and r["result"]["dtype"] == "f32"
    return r["result"]["tensor_id"]


@pytest.mark.gpu
def test_tensor_matmul_vectors_on_gpu(primal):
    """sprint56b_tests.rs:618-669 ([[1,2],[3,4]].[[5,6],[7,8]] = [[19,22],[43,50]];
    [1,0,2].[1,0,3]^T = 7) and tensor_fhe_tests.rs's 2x3.3x2 = [[58,64],[139,154]],
    through tensor.create + tensor.matmul (bch_sgemm)."""
    print("ipc tensor.matmul vectors", flush=True)
    cases = [([2, 2], [1, 2, 3, 4], [2, 2], [5, 6, 7, 8], [19, 22, 43, 50]),
             ([1, 3], [1, 0, 2], [3, 1], [1, 0, 3], [7]),
             ([2, 3], [1, 2, 3, 4, 5, 6], [3, 2], [7, 8, 9, 10, 11, 12], [58, 64, 139, 154])]
    for i, (sa, a, sb, b, want) in enumerate(cases):
        la, lb = _create(primal, sa, a, 100 + i), _create(primal, sb, b, 200 + i)
        r = ipc.dispatch(primal, "barracuda.tensor.matmul", {"lhs_id": la, "rhs_id": lb}, 300 + i)
        res = r["result"]
        assert res["status"] == "completed" and res["shape"] == [sa[0], sb[1]] and res["elements"] == len(want)
        got = primal.get_tensor(res["result_id"]).to_vec()
        assert got.tolist() == want
    # shape errors come back as the reference's Matmul failed / INTERNAL_ERROR
    la, lb = _create(primal, [2, 3], [1] * 6, 400), _create(primal, [2, 3], [1] * 6, 401)
    e = _err(ipc.tensor_matmul(primal, {"lhs_id": la, "rhs_id": lb}, 402))
    assert e["code"] == ipc.INTERNAL_ERROR and e["message"].startswith("Matmul failed: ") and "mismatch" in e["message"]


@pytest.mark.gpu
def test_batch_submit_wire_contract_example(primal):
    """The request/response example of batch.rs:8-37."""
    print("ipc tensor.batch.submit wire example", flush=True)
    r = ipc.dispatch(primal, "tensor.batch.submit", {"ops": [
        {"op": "create", "alias": "x", "data": [1, 2, 3, 4], "shape": [1, 4]},
        {"op": "create", "alias": "w", "data": [1, 0, 0, 1], "shape": [4, 1]},
        {"op": "matmul", "alias": "h", "a": "x", "b": "w"},
        {"op": "relu", "alias": "out", "input": "h"},
        {"op": "readback", "alias": "final", "input": "out"}]}, 1)
    res = r["result"]
    assert res["status"] == "completed" and res["ops_executed"] == 5
    out = res["outputs"]
    assert out["final"] == {"data": [5.0], "shape": [1, 1]}
    assert out["x"]["shape"] == [1, 4] and out["x"]["elements"] == 4
    assert out["h"]["shape"] == [1, 1] and out["out"]["elements"] == 1
    for k in ("x", "w", "h", "out"):
        assert primal.get_tensor(out[k]["result_id"]) is not None
    assert primal.get_tensor(out["out"]["result_id"]).to_vec().tolist() == [5.0]


@pytest.mark.gpu
def test_batch_submit_every_op_against_oracle(primal):
    """One request over every batch op; the readbacks against numpy / the f64 oracle."""
    print("ipc tensor.batch.submit every op", flush=True)
    r = O.Lcg(55)
    a, b, c = r.normal((8, 64)), r.normal((8, 64)), r.normal((8, 64))
    w = r.normal((64, 32), 0.0, 0.2)
    L = lambda x: x.reshape(-1).astype(float).tolist()
    ops = [{"op": "create", "alias": "a", "shape": [8, 64], "data": L(a)},
           {"op": "create", "alias": "b", "shape": [8, 64], "data": L(b)},
           {"op": "create", "alias": "c", "shape": [8, 64], "data": L(c)},
           {"op": "create", "alias": "w", "shape": [64, 32], "data": L(w)},
           {"op": "add", "alias": "s", "a": "a", "b": "b"},
           {"op": "sub", "alias": "d", "a": "a", "b": "b"},
           {"op": "mul", "alias": "p", "a": "a", "b": "b"},
           {"op": "negate", "alias": "n", "input": "a"},
           {"op": "fma", "alias": "f", "a": "a", "b": "b", "c": "c"},
           {"op": "scale", "alias": "sc", "input": "a", "scalar": 0.5},
           {"op": "matmul", "alias": "h", "a": "s", "b": "w"},
           {"op": "gelu", "alias": "g", "input": "h"},
           {"op": "layer_norm", "alias": "ln", "input": "g", "feature_size": 32},
           {"op": "reshape", "alias": "flat", "input": "ln", "shape": [256]},
           {"op": "softmax", "alias": "sm", "input": "flat"},
           {"op": "readback", "alias": "", "input": "sm"},
           {"op": "readback", "alias": "rb_ln", "input": "ln"},
           {"op": "readback", "alias": "rb_f", "input": "f"},
           {"op": "readback", "alias": "rb_n", "input": "n"}]
    res = ipc.tensor_batch_submit(primal, {"ops": ops}, 77)["result"]
    assert res["ops_executed"] == len(ops)
    out = res["outputs"]
    hv = (a + b).astype(np.float64) @ w.astype(np.float64)
    g = 0.5 * hv * (1.0 + np.tanh(0.7978845608 * (hv + 0.044715 * hv ** 3)))
    ln = (g - g.mean(axis=1, keepdims=True)) / np.sqrt(g.var(axis=1, keepdims=True) + 1e-5)
    assert out["rb_ln"]["shape"] == [8, 32]
    assert O.max_rel_err(np.array(out["rb_ln"]["data"], np.float32), ln.reshape(-1)) <= TOL
    e = np.exp(ln.reshape(-1) - ln.max())
    assert O.max_rel_err(np.array(out["sm"]["data"], np.float32), e / e.sum()) <= TOL  # readback under its input alias
    assert np.array_equal(np.array(out["rb_n"]["data"], np.float32), (-a).reshape(-1))
    exact = (a.astype(np.float64) * b + c).reshape(-1)
    assert np.max(np.abs(np.array(out["rb_f"]["data"]) - exact) / np.maximum(np.abs(exact), 1e-30)) < 1.2e-7
    assert out["flat"]["shape"] == [256] and out["sc"]["elements"] == 512
    # a session-level error is INVALID_PARAMS with the op index
    bad = ipc.tensor_batch_submit(primal, {"ops": [
        {"op": "create", "alias": "x", "shape": [2, 3]}, {"op": "create", "alias": "y", "shape": [3, 2]},
        {"op": "add", "alias": "z", "a": "x", "b": "y"}]}, 78)
    e = _err(bad)
    assert e["code"] == ipc.INVALID_PARAMS and e["message"] == "ops[2]: Shape mismatch: expected [2, 3], got [3, 2]"
    bad = ipc.tensor_batch_submit(primal, {"ops": [
        {"op": "create", "alias": "x", "shape": [2, 3]},
        {"op": "layer_norm", "alias": "y", "input": "x", "feature_size": 4}]}, 79)
    assert _err(bad)["message"] == "ops[1]: layer_norm failed: Invalid input: layer_norm: total 6 not divisible by feature_size 4"


@pytest.mark.gpu
def test_inline_f64_handlers_golden_on_gpu(primal, golden):
    """sprint56b_tests.rs:618-669 and ml_tests.rs:128-165 through dispatch
    (bch_dgemm; bch_dgemm + bch_softmax_rows_f64 + bch_dgemm)."""
    print("ipc inline f64 handlers: reference vectors", flush=True)
    for i, case in enumerate(golden["inline_f64"]):
        r = ipc.dispatch(primal, case["method"], case["params"], 500 + i)
        assert "result" in r, (case["name"], r)
        got = np.array(r["result"]["result"], dtype=np.float64)
        want = np.array(case["expected"])
        assert got.shape == want.shape, case["name"]
        assert np.max(np.abs(got - want)) <= case["tol"] * max(1.0, np.max(np.abs(want))), case["name"]
        if case["method"] == "tensor.matmul_inline":
            assert r["result"]["shape"] == case["shape"]
        else:
            q, k, v = (case["params"][x] for x in "qkv")
            assert (r["result"]["seq_q"], r["result"]["seq_k"], r["result"]["d_k"], r["result"]["d_v"]) == \
                (len(q), len(k), len(q[0]), len(v[0]))


@pytest.mark.gpu
def test_inline_f64_handlers_vs_oracle_on_gpu(primal):
    """Seeded inline data against the f64 restatements of the handlers'
    loops (ml/forward.rs:121-150, tensor.rs:540-548): max |x - ref| /
    max(|ref|, 1) <= 1e-12 (f64 against f64; only the summation order
    differs).  Includes one-row, one-key, d_v = 0 and 300-key cases."""
    print("ipc inline f64 handlers vs oracle", flush=True)
    rng = O.Lcg(31)
    for sq, sk, dk, dv in ((1, 1, 1, 1), (5, 3, 4, 2), (37, 300, 24, 17), (64, 64, 64, 64), (3, 2049, 8, 5),
                           (2, 7, 3, 0)):
        q, k, v = (rng.normal(s).astype(np.float64) for s in ((sq, dk), (sk, dk), (sk, dv)))
        params = {"q": q.tolist(), "k": k.tolist(), "v": v.tolist() if dv else [[] for _ in range(sk)]}
        r = ipc.dispatch(primal, "ml.attention", params, 600)
        assert "result" in r, r
        got = np.array(r["result"]["result"], dtype=np.float64).reshape(sq, dv)
        want = O.ml_attention_f64(q, k, v)
        assert np.max(np.abs(got - want), initial=0.0) <= 1e-12 * max(1.0, np.max(np.abs(want), initial=0.0)), \
            (sq, sk, dk, dv)
    for m, k_, n in ((1, 1, 1), (7, 13, 5), (33, 100, 65), (128, 64, 3)):
        a, b = rng.normal((m, k_)).astype(np.float64), rng.normal((k_, n)).astype(np.float64)
        r = ipc.dispatch(primal, "tensor.matmul_inline", {"lhs": a.tolist(), "rhs": b.tolist()}, 700)
        assert r["result"]["shape"] == [m, n]
        got = np.array(r["result"]["result"], dtype=np.float64)
        want = O.matmul_inline_f64(a, b)
        assert np.max(np.abs(got - want)) <= 1e-12 * max(1.0, np.max(np.abs(want))), (m, k_, n)
    r = ipc.dispatch(primal, "tensor.matmul_inline", {"lhs": [[1.0, 2.0]], "rhs": [[], []]}, 701)
    assert r["result"] == {"result": [[]], "shape": [1, 0]}
    # scores that overflow to inf: inf - inf in the softmax, NaN weights, null outputs (serde_json)
    r = ipc.dispatch(primal, "ml.attention", {"q": [[1e200]], "k": [[1e200], [1.0]], "v": [[1.0], [2.0]]}, 702)
    assert r["result"]["result"] == [[None]]
