"""JSON-RPC method handlers of the tensor wire paths, routed to the HIP path.

Mirrors, at the handler level only, crates/barracuda-core/src/ipc/ of the
reference (no server, transport, method gate or BTSP: those are the
reference's control plane):

  normalize_method                    ipc/methods/mod.rs:173-180
  dispatch (the tensor routes)        ipc/methods/mod.rs:210-355
  tensor.create                       ipc/methods/tensor.rs:32-116
  tensor.matmul                       ipc/methods/tensor.rs:118-168
  tensor.batch.submit                 ipc/methods/batch.rs:58-283
  batch pre-validation                ipc/methods/batch.rs:287-350
  batch op helpers                    ipc/methods/batch.rs:352-537
  tensor.matmul_inline                ipc/methods/tensor.rs:490-552
  ml.attention                        ipc/methods/ml/forward.rs:80-165
  extract_matrix                      ipc/methods/params.rs:21-30
  JSON-RPC error codes                ipc/jsonrpc.rs:51-59
  parse_shape                         ipc/methods/compute.rs:16-22

Each handler takes the params object exactly as the reference handler reads
it and returns the same response object ({"jsonrpc", "result" | "error",
"id"}), with the same validation order, error codes and message wording.
The compute runs on the HIP path: tensor.matmul calls Tensor.matmul_ref
(bch_sgemm) and tensor.batch.submit records and runs a TensorSession
(bch_sgemm, bch_elementwise, bch_softmax_rows, bch_layer_norm).  The two
inline-data handlers compute in f64, as the reference's do:
tensor.matmul_inline on bch_dgemm, ml.attention on bch_dgemm (Q K^T, scaled)
-> bch_softmax_rows_f64 -> bch_dgemm (P V).  Non-finite result values are
written as null, as serde_json writes a non-finite f64.

Deliberate difference: the reference keeps a CPU tensor store for headless
hosts (CpuTensor, tensor.rs:97-114, 158-167).  This path has no CPU
fallback: without a device, tensor.create answers INTERNAL_ERROR "No GPU
device available", as tensor.batch.submit already does in the reference
(batch.rs:95-97), and tensor.matmul finds no stored tensor ("Tensor not
found", INVALID_PARAMS, the reference's answer for unknown ids).  The same
holds for ml.attention and tensor.matmul_inline, which the reference computes
on the host: their validation answers are unchanged, and a valid request
without a device answers INTERNAL_ERROR "No GPU device available".
"""
from __future__ import annotations

import hashlib
import itertools
import threading
from typing import Any

import numpy as np

from .error import BarracudaError
from .linalg import GemmF64, attention_f64
from .session import SessionTensor, TensorSession
from .tensor import HipDevice, Tensor

__all__ = ["PARSE_ERROR", "INVALID_REQUEST", "METHOD_NOT_FOUND", "INVALID_PARAMS", "INTERNAL_ERROR",
           "PRIMAL_NAMESPACE", "TensorPrimal", "normalize_method", "dispatch", "tensor_create",
           "tensor_matmul", "tensor_matmul_inline", "tensor_batch_submit", "ml_attention", "ROUTED_METHODS"]

# ipc/jsonrpc.rs:51-59
PARSE_ERROR = -32700
INVALID_REQUEST = -32600
METHOD_NOT_FOUND = -32601
INVALID_PARAMS = -32602
INTERNAL_ERROR = -32603
JSONRPC_VERSION = "2.0"
PRIMAL_NAMESPACE = "barracuda"  # barracuda-core/src/lib.rs:130

_U64_MAX = 2**64 - 1


def _success(id_: Any, result: Any) -> dict:
    """JsonRpcResponse::success (jsonrpc.rs:66-73)."""
    return {"jsonrpc": JSONRPC_VERSION, "result": result, "id": id_}


def _error(id_: Any, code: int, message: str) -> dict:
    """JsonRpcResponse::error (jsonrpc.rs:76-87)."""
    return {"jsonrpc": JSONRPC_VERSION, "error": {"code": code, "message": message}, "id": id_}


def _is_u64(v: Any) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and 0 <= v <= _U64_MAX


def _as_f64(v: Any):
    """serde_json Value::as_f64: numbers only (bool is not a number)."""
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    return float(v)


def _json_num(x: float):
    """serde_json's Value for an f64: a number, or null when not finite."""
    x = float(x)
    return x if np.isfinite(x) else None


def _extract_matrix(params: dict, key: str):
    """params.rs:21-30 extract_matrix: the array rows of params[key] (rows
    that are not arrays are dropped), each row's numeric entries (others
    dropped); None when params[key] is not an array."""
    rows = params.get(key)
    if not isinstance(rows, list):
        return None
    return [[x for x in (_as_f64(c) for c in row) if x is not None] for row in rows if isinstance(row, list)]


def _parse_shape(arr: list) -> list[int]:
    """compute.rs:16-22: the u64 entries of the array (others are skipped);
    every u64 fits a 64-bit usize."""
    return [int(v) for v in arr if _is_u64(v)]


def _f32_data(arr: list) -> np.ndarray:
    """The numeric entries of a JSON array as f32 (f64 -> f32 narrowing, as
    the reference's `n as f32`); non-numbers are skipped."""
    vals = [x for x in (_as_f64(v) for v in arr) if x is not None]
    return np.asarray(vals, dtype=np.float64).astype(np.float32)


class TensorPrimal:
    """The part of BarraCudaPrimal (barracuda-core/src/lib.rs) the tensor
    handlers use: the device (None on a host without one) and the tensor
    store, keyed by 16 hex characters as store_tensor does (lib.rs:261-272)."""

    def __init__(self, device: HipDevice | None):
        self._device = device
        self._tensors: dict[str, Tensor] = {}
        self._lock = threading.Lock()
        self._count = itertools.count()

    def device(self) -> HipDevice | None:
        return self._device

    def store_tensor(self, tensor: Tensor) -> str:
        with self._lock:
            key = hashlib.blake2b(f"{id(tensor):x}:{next(self._count)}".encode(), digest_size=8).hexdigest()
            self._tensors[key] = tensor
        return key

    def get_tensor(self, key: str) -> Tensor | None:
        with self._lock:
            return self._tensors.get(key)

    def tensor_count(self) -> int:
        with self._lock:
            return len(self._tensors)


def normalize_method(method: str) -> str:
    """mod.rs:173-180: `barracuda.tensor.matmul` -> `tensor.matmul`."""
    prefix = PRIMAL_NAMESPACE + "."
    return method[len(prefix):] if method.startswith(prefix) else method


def tensor_create(primal: TensorPrimal, params: dict, id_: Any) -> dict:
    """tensor.rs:32-116: validate shape and data, then upload to the device."""
    shape = params.get("shape") if isinstance(params, dict) else None
    if not isinstance(shape, list):
        return _error(id_, INVALID_PARAMS, "Missing required param: shape")
    shape_vec = _parse_shape(shape)
    elements = int(np.prod(shape_vec, dtype=object)) if shape_vec else 1
    data_arr = params.get("data")
    data = _f32_data(data_arr) if isinstance(data_arr, list) else np.zeros(elements, np.float32)
    if data.size != elements:
        return _error(id_, INVALID_PARAMS, f"data length {data.size} does not match shape product {elements}")
    dev = primal.device()
    if dev is None:
        return _error(id_, INTERNAL_ERROR, "No GPU device available")
    try:
        tensor = Tensor.from_data(data, shape_vec, dev)
    except BarracudaError as e:
        return _error(id_, INTERNAL_ERROR, f"Tensor creation failed: {e}")
    tid = primal.store_tensor(tensor)
    return _success(id_, {"status": "completed", "tensor_id": tid, "result_id": tid, "shape": shape_vec,
                          "elements": elements, "dtype": "f32"})


def tensor_matmul(primal: TensorPrimal, params: dict, id_: Any) -> dict:
    """tensor.rs:118-168: lhs.matmul_ref(rhs) of two stored tensors, the
    product stored and described."""
    lhs_id = params.get("lhs_id") if isinstance(params, dict) else None
    if not isinstance(lhs_id, str):
        return _error(id_, INVALID_PARAMS, "Missing required param: lhs_id")
    rhs_id = params.get("rhs_id")
    if not isinstance(rhs_id, str):
        return _error(id_, INVALID_PARAMS, "Missing required param: rhs_id")
    lhs = primal.get_tensor(lhs_id)
    if lhs is None:
        return _error(id_, INVALID_PARAMS, f"Tensor not found: {lhs_id}")
    rhs = primal.get_tensor(rhs_id)
    if rhs is None:
        return _error(id_, INVALID_PARAMS, f"Tensor not found: {rhs_id}")
    try:
        result = lhs.matmul_ref(rhs)
    except BarracudaError as e:
        return _error(id_, INTERNAL_ERROR, f"Matmul failed: {e}")
    shape = result.shape()
    rid = primal.store_tensor(result)
    return _success(id_, {"status": "completed", "result_id": rid, "shape": shape,
                          "elements": int(np.prod(shape, dtype=object)) if shape else 1})


# ---- tensor.batch.submit ----------------------------------------------------------------
VALID_OPS = ("create", "add", "sub", "mul", "negate", "fma", "scale", "matmul", "relu", "gelu", "softmax",
             "layer_norm", "reshape", "readback")


class _BatchError(Exception):
    """batch.rs:46-56 BatchError: its message is the response message."""


def _validate_batch_ops(ops: list) -> None:
    """batch.rs:287-350: everything that can be checked before a device is
    needed, in op order."""
    defined: set[str] = set()
    for i, op in enumerate(ops):
        name = op.get("op") if isinstance(op, dict) else None
        if not isinstance(name, str):
            raise _BatchError(f"ops[{i}]: missing 'op' field")
        if name not in VALID_OPS:
            raise _BatchError(f"ops[{i}]: unknown op '{name}'")
        alias = op.get("alias")
        if isinstance(alias, str) and alias:
            defined.add(alias)
        if name == "create":
            shape = op.get("shape")
            if not isinstance(shape, list):
                raise _BatchError(f"ops[{i}]: create requires 'shape'")
            data = op.get("data")
            if isinstance(data, list):
                elements = 1
                for v in shape:
                    if _is_u64(v):
                        elements = min(elements * v, _U64_MAX)
                if len(data) != elements:
                    raise _BatchError(f"ops[{i}]: data length {len(data)} ≠ shape product {elements}")
        elif name == "readback":
            src = op.get("input")
            if not isinstance(src, str):
                raise _BatchError(f"ops[{i}]: readback requires 'input' alias")
            if src not in defined:
                raise _BatchError(f"ops[{i}]: unknown alias '{src}'")
        elif name in ("add", "sub", "mul", "matmul", "fma"):
            for key in (("a", "b", "c") if name == "fma" else ("a", "b")):
                ref = op.get(key)
                if not isinstance(ref, str):
                    raise _BatchError(f"ops[{i}]: {name} requires '{key}' alias")
                if ref not in defined:
                    raise _BatchError(f"ops[{i}]: unknown alias '{ref}'")
        else:  # scale relu gelu softmax negate layer_norm reshape
            ref = op.get("input")
            if not isinstance(ref, str):
                raise _BatchError(f"ops[{i}]: {name} requires 'input' alias")
            if ref not in defined:
                raise _BatchError(f"ops[{i}]: unknown alias '{ref}'")
            if name == "scale" and _as_f64(op.get("scalar")) is None:
                raise _BatchError(f"ops[{i}]: scale requires 'scalar'")
            if name == "layer_norm" and not _is_u64(op.get("feature_size")):
                raise _BatchError(f"ops[{i}]: layer_norm requires 'feature_size'")
            if name == "reshape" and not isinstance(op.get("shape"), list):
                raise _BatchError(f"ops[{i}]: reshape requires 'shape'")


def _resolve(aliases: dict, op: dict, key: str, idx: int) -> SessionTensor:
    """batch.rs:367-380."""
    name = op.get(key)
    if not isinstance(name, str):
        raise _BatchError(f"ops[{idx}]: missing '{key}' alias")
    if name not in aliases:
        raise _BatchError(f"ops[{idx}]: unknown alias '{name}'")
    return aliases[name]


def _record(session: TensorSession, aliases: dict, op: dict, idx: int, name: str) -> SessionTensor:
    """batch.rs:382-537: record one op in the session."""
    try:
        if name == "create":
            shape = _parse_shape(op["shape"])
            elements = int(np.prod(shape, dtype=object)) if shape else 1
            data = _f32_data(op["data"]) if isinstance(op.get("data"), list) else np.zeros(elements, np.float32)
            if data.size != elements:
                raise _BatchError(f"ops[{idx}]: data length {data.size} ≠ shape product {elements}")
            try:
                return session.tensor_with_shape(data, shape)
            except BarracudaError as e:
                raise _BatchError(f"ops[{idx}]: create failed: {e}") from e
        if name in ("add", "sub", "mul", "matmul"):
            a, b = _resolve(aliases, op, "a", idx), _resolve(aliases, op, "b", idx)
            return getattr(session, name)(a, b)
        if name == "fma":
            a, b, c = (_resolve(aliases, op, k, idx) for k in ("a", "b", "c"))
            try:
                return session.fma(a, b, c)
            except BarracudaError as e:
                raise _BatchError(f"ops[{idx}]: fma failed: {e}") from e
        if name == "scale":
            a = _resolve(aliases, op, "input", idx)
            scalar = _as_f64(op.get("scalar"))
            if scalar is None:
                raise _BatchError(f"ops[{idx}]: scale requires 'scalar'")
            try:
                return session.scale(a, float(np.float32(scalar)))
            except BarracudaError as e:
                raise _BatchError(f"ops[{idx}]: scale failed: {e}") from e
        if name in ("relu", "gelu", "softmax", "negate"):
            return getattr(session, name)(_resolve(aliases, op, "input", idx))
        if name == "layer_norm":
            a = _resolve(aliases, op, "input", idx)
            fs = op.get("feature_size")
            if not _is_u64(fs):
                raise _BatchError(f"ops[{idx}]: layer_norm requires 'feature_size'")
            try:
                return session.layer_norm(a, fs)
            except BarracudaError as e:
                raise _BatchError(f"ops[{idx}]: layer_norm failed: {e}") from e
        if name == "reshape":
            a = _resolve(aliases, op, "input", idx)
            shape = op.get("shape")
            if not isinstance(shape, list):
                raise _BatchError(f"ops[{idx}]: reshape requires 'shape'")
            try:
                return session.reshape(a, _parse_shape(shape))
            except BarracudaError as e:
                raise _BatchError(f"ops[{idx}]: reshape failed: {e}") from e
    except BarracudaError as e:  # the binary and unary ops' own errors
        raise _BatchError(f"ops[{idx}]: {e}") from e
    raise _BatchError(f"ops[{idx}]: unknown op '{name}'")


def tensor_batch_submit(primal: TensorPrimal, params: dict, id_: Any) -> dict:
    """batch.rs:58-283: validate, record every op in one TensorSession, run
    it as one batch on the device's stream, then store every aliased tensor
    and read back the requested ones."""
    ops = params.get("ops") if isinstance(params, dict) else None
    if not isinstance(ops, list):
        return _error(id_, INVALID_PARAMS, "Missing required param: ops (array of batch operations)")
    if not ops:
        return _error(id_, INVALID_PARAMS, "ops array must not be empty")
    try:
        _validate_batch_ops(ops)
    except _BatchError as e:
        return _error(id_, INVALID_PARAMS, str(e))
    dev = primal.device()
    if dev is None:
        return _error(id_, INTERNAL_ERROR, "No GPU device available")
    session = TensorSession.with_device(dev)
    aliases: dict[str, SessionTensor] = {}
    readbacks: list[tuple[str, str]] = []
    for i, op in enumerate(ops):
        name = op.get("op")
        if not isinstance(name, str):
            return _error(id_, INVALID_PARAMS, f"ops[{i}]: missing 'op' field")
        alias = op.get("alias") if isinstance(op.get("alias"), str) else ""
        if name == "readback":
            src = op.get("input")
            if not isinstance(src, str):
                return _error(id_, INVALID_PARAMS, f"ops[{i}]: readback missing 'input' alias")
            readbacks.append((alias, src))
            continue
        try:
            t = _record(session, aliases, op, i, name)
        except _BatchError as e:
            return _error(id_, INVALID_PARAMS, str(e))
        if alias:
            aliases[alias] = t
    try:
        session.run()
    except BarracudaError as e:
        return _error(id_, INTERNAL_ERROR, f"Batch execution failed: {e}")
    outputs: dict[str, Any] = {}
    for alias, t in aliases.items():
        shape = t.shape()
        try:
            stored = t.to_tensor()
        except BarracudaError as e:
            return _error(id_, INTERNAL_ERROR, f"Failed to export tensor '{alias}': {e}")
        outputs[alias] = {"result_id": primal.store_tensor(stored), "shape": shape, "elements": t.len()}
    for rb_alias, src in readbacks:
        t = aliases.get(src)
        if t is None:
            return _error(id_, INTERNAL_ERROR, f"readback: alias '{src}' lost after execution")
        try:
            data = t.to_vec()
        except BarracudaError as e:
            return _error(id_, INTERNAL_ERROR, f"Readback of '{src}' failed: {e}")
        outputs[rb_alias or src] = {"data": [_json_num(x) for x in data], "shape": t.shape()}
    return _success(id_, {"status": "completed", "outputs": outputs, "ops_executed": len(ops)})


# ---- inline-data f64 handlers -------------------------------------------------------------
def tensor_matmul_inline(primal: TensorPrimal, params: dict, id_: Any) -> dict:
    """tensor.rs:490-552: lhs [m x k] times rhs [k x n] sent inline, the
    product returned inline (f64, on bch_dgemm)."""
    lhs = _extract_matrix(params, "lhs") if isinstance(params, dict) else None
    rhs = _extract_matrix(params, "rhs") if isinstance(params, dict) else None
    if lhs is None or rhs is None:
        return _error(id_, INVALID_PARAMS, "Missing required params: lhs and rhs (2D arrays)")
    m = len(lhs)
    if m == 0:
        return _error(id_, INVALID_PARAMS, "lhs must be non-empty")
    k = len(lhs[0])
    if k == 0 or any(len(r) != k for r in lhs):
        return _error(id_, INVALID_PARAMS, "lhs rows must have consistent length")
    if not rhs:
        return _error(id_, INVALID_PARAMS, "rhs must be non-empty")
    n = len(rhs[0])
    if len(rhs) != k or any(len(r) != n for r in rhs):
        return _error(id_, INVALID_PARAMS, f"Shape mismatch: lhs is [{m}x{k}], rhs must be [{k}x{n}]")
    dev = primal.device()
    if dev is None:
        return _error(id_, INTERNAL_ERROR, "No GPU device available")
    if n == 0:
        return _success(id_, {"result": [[] for _ in range(m)], "shape": [m, n]})
    try:
        c = GemmF64.execute(dev, np.asarray(lhs, dtype=np.float64), np.asarray(rhs, dtype=np.float64), m, k, n, 1)
    except BarracudaError as e:
        return _error(id_, INTERNAL_ERROR, f"Matmul failed: {e}")
    result = [[_json_num(x) for x in row] for row in c.reshape(m, n)]
    return _success(id_, {"result": result, "shape": [m, n]})


def ml_attention(primal: TensorPrimal, params: dict, id_: Any) -> dict:
    """ml/forward.rs:80-165: softmax(Q K^T / sqrt(d_k)) V on inline 2-D q, k,
    v (f64: bch_dgemm, bch_softmax_rows_f64, bch_dgemm)."""
    if not isinstance(params, dict):
        params = {}
    q = _extract_matrix(params, "q")
    if q is None:
        return _error(id_, INVALID_PARAMS, "Missing required param: q (2D array)")
    k = _extract_matrix(params, "k")
    if k is None:
        return _error(id_, INVALID_PARAMS, "Missing required param: k (2D array)")
    v = _extract_matrix(params, "v")
    if v is None:
        return _error(id_, INVALID_PARAMS, "Missing required param: v (2D array)")
    if not q or not k or not v:
        return _error(id_, INVALID_PARAMS, "q, k, v must be non-empty")
    d_k = len(q[0])
    if d_k == 0:
        return _error(id_, INVALID_PARAMS, "Key dimension must be > 0")
    seq_q, seq_k = len(q), len(k)
    if any(len(r) != d_k for r in k) or any(len(r) != d_k for r in q):
        return _error(id_, INVALID_PARAMS, "q and k must have matching inner dimension")
    d_v = len(v[0])
    if len(v) != seq_k or any(len(r) != d_v for r in v):
        return _error(id_, INVALID_PARAMS, "v must have same sequence length as k with consistent column count")
    dev = primal.device()
    if dev is None:
        return _error(id_, INTERNAL_ERROR, "No GPU device available")
    try:
        out = attention_f64(dev, np.asarray(q, dtype=np.float64), np.asarray(k, dtype=np.float64),
                            np.asarray(v, dtype=np.float64).reshape(seq_k, d_v))
    except BarracudaError as e:
        return _error(id_, INTERNAL_ERROR, f"Attention failed: {e}")
    return _success(id_, {"result": [[_json_num(x) for x in row] for row in out], "seq_q": seq_q,
                          "seq_k": seq_k, "d_k": d_k, "d_v": d_v})


# method name -> handler (mod.rs:315-338, the routes this path serves)
ROUTED_METHODS = {
    "tensor.create": tensor_create,
    "tensor.matmul": tensor_matmul,
    "tensor.matmul_inline": tensor_matmul_inline,
    "tensor.batch.submit": tensor_batch_submit,
    "ml.attention": ml_attention,
}


def dispatch(primal: TensorPrimal, method: str, params: Any, id_: Any) -> dict:
    """mod.rs:210-355 for the routed tensor methods; any other method is
    METHOD_NOT_FOUND "Unknown method: <method>" (mod.rs:355)."""
    handler = ROUTED_METHODS.get(normalize_method(method))
    if handler is None:
        return _error(id_, METHOD_NOT_FOUND, f"Unknown method: {method}")
    return handler(primal, params if isinstance(params, dict) else {}, id_)
