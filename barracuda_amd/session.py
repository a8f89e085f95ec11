"""TensorSession: record ops, then run them in one batch.

Mirrors crates/barracuda/src/session/:
  AttentionDims {batch_size, n_heads, seq_len, head_dim}   session/mod.rs:60-99
  TensorSession::{new, with_device, reset, num_ops}        session/mod.rs:134-165
  TensorSession::{tensor, tensor_with_shape, import}       session/mod.rs:172-207
  TensorSession::{add, sub, mul, negate, fma, scale}       session/mod.rs:214-300
  TensorSession::matmul                                    session/mod.rs:305-333
  TensorSession::{relu, gelu}                              session/mod.rs:340-360
  TensorSession::softmax                                   session/mod.rs:364-371
  TensorSession::layer_norm                                session/mod.rs:379-398
  TensorSession::reshape                                   session/mod.rs:403-415
  TensorSession::{head_split, head_concat}                 session/mod.rs:423-480
  TensorSession::attention                                 session/mod.rs:481-518
  TensorSession::run                                       session/mod.rs:521-540
  SessionTensor::{shape, len, is_empty, to_vec, to_tensor} session/tensor.rs:14-68

Recording allocates the output buffer in HBM (zero-filled, as a fresh wgpu
buffer is) and appends the op; nothing is launched until `run()`, which
enqueues every recorded op, in order, on the device's one stream and then
waits once.  Ops read each other's outputs in recording order, which the
single in-order stream guarantees without extra synchronisation.

Each op routes to the kernels of this package, with launch grids that cover
the whole problem.  This deliberately does not reproduce three dispatch
defects of the reference session:
  * matmul tiers Tiled16 / GpuEvolved32 launch (ceil(m/16), ceil(n/16))
    workgroups while the shaders map x to columns (session/types.rs:53-58),
    so non-square results come back incomplete;
  * softmax launches one workgroup of the global-softmax shader
    (session/dispatch.rs:217), so only the first 256 outputs are written;
  * attention dispatches B*H*S^2 / 256 workgroups (dispatch.rs:289-295),
    over the 65,535 limit at S = 2048.
softmax is the global softmax over every element of the input, which is
what the shader the reference session binds (softmax_simple_f64.wgsl)
computes for each output it writes; attention is the non-causal
softmax(Q K^T / sqrt(D)) V over [B, H, S, D].

The element-wise ops, ReLU and GELU run on bch_elementwise; layer_norm on
bch_layer_norm with the epsilon the reference session passes (1e-5,
dispatch.rs:221-240).  head_split / head_concat move [B, S, H*D] <-> [B, H, S, D]
on bch_head_split / bch_head_concat (an HBM-streaming permutation, bit-exact),
so the reference's recipe -- projection matmul, head_split, attention,
head_concat, output matmul -- runs as recorded.  attention takes any head_dim.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from .error import CastOverflow, ExecutionError, InvalidInput, InvalidShape, ShapeMismatch, UnsupportedOperation
from . import _native as N
from .tensor import HipDevice, Tensor, _Buffer, _check_i32, _numel, get_device

__all__ = ["AttentionDims", "SessionTensor", "TensorSession"]

_U32_MAX = 2**32 - 1
LAYER_NORM_EPS = 1e-5  # session/dispatch.rs:221-240

# session op name -> (BCH_EW_* code, operands read)
_ELEMENTWISE = {"add": (N.BCH_EW_ADD, 2), "sub": (N.BCH_EW_SUB, 2), "mul": (N.BCH_EW_MUL, 2),
                "negate": (N.BCH_EW_NEG, 1), "fma": (N.BCH_EW_FMA, 3), "scale": (N.BCH_EW_SCALE, 1),
                "relu": (N.BCH_EW_RELU, 1), "gelu": (N.BCH_EW_GELU, 1)}


def _usize_as_u32(v: int) -> int:
    """cast.rs:31-37 usize_as_u32."""
    if v > _U32_MAX:
        raise CastOverflow("usize", "u32", f"{v}")
    return v


@dataclass(frozen=True)
class AttentionDims:
    """session/mod.rs:60-99: the [B, H, S, D] dimensions of an attention op."""

    batch_size: int
    n_heads: int
    seq_len: int
    head_dim: int

    def total_elements(self) -> int:
        """B x H x S x D (session/mod.rs:78-81)."""
        return self.batch_size * self.n_heads * self.seq_len * self.head_dim

    def as_u32(self) -> tuple[int, int, int, int]:
        """(batch_size, seq_len, n_heads, head_dim), each checked to fit u32
        (session/mod.rs:91-98)."""
        return (_usize_as_u32(self.batch_size), _usize_as_u32(self.seq_len),
                _usize_as_u32(self.n_heads), _usize_as_u32(self.head_dim))


class SessionTensor:
    """session/tensor.rs:14-68: a buffer owned by a session, with its shape.

    The buffer exists from the moment the tensor is created; an op's output
    reads as zeros until `TensorSession.run()` has executed the op."""

    __slots__ = ("_session", "buffer_id", "_shape")

    def __init__(self, session: "TensorSession", buffer_id: int, shape: Sequence[int]):
        self._session = session
        self.buffer_id = buffer_id
        self._shape = [int(s) for s in shape]

    def shape(self) -> list[int]:
        return list(self._shape)

    def len(self) -> int:
        return _numel(self._shape)

    def is_empty(self) -> bool:
        return self.len() == 0

    @property
    def ptr(self) -> int:
        return self._session._buffers[self.buffer_id].ptr

    def to_vec(self) -> np.ndarray:
        """Blocking readback of the flat f32 contents (tensor.rs:49-55)."""
        buf = self._session._buffers[self.buffer_id]
        if buf.nbytes == 0:
            return np.empty(0, dtype=np.float32)
        return self._session.device.download(buf.ptr, buf.nbytes)

    def to_tensor(self) -> Tensor:
        """A standalone Tensor holding a copy (tensor.rs:64-67)."""
        return Tensor.from_data(self.to_vec(), self._shape, self._session.device)


class TensorSession:
    """session/mod.rs:118-540: ops are recorded, then executed by `run()`."""

    def __init__(self, device: HipDevice | None = None):
        self.device = device or get_device()
        self._buffers: list[_Buffer] = []
        self._shapes: list[list[int]] = []
        self._ops: list[tuple] = []
        self.executed = False

    @classmethod
    def new(cls, device: HipDevice | None = None) -> "TensorSession":
        return cls(device)

    @classmethod
    def with_device(cls, device: HipDevice) -> "TensorSession":
        return cls(device)

    def reset(self) -> None:
        """Clear recorded ops; buffers stay allocated (session/mod.rs:155-158)."""
        self._ops.clear()
        self.executed = False

    def num_ops(self) -> int:
        return len(self._ops)

    # -- input ingestion ---------------------------------------------------
    def tensor(self, data) -> SessionTensor:
        """Upload a flat slice as a 1-D tensor (session/mod.rs:172-174)."""
        arr = np.asarray(data, dtype=np.float32).reshape(-1)
        return self.tensor_with_shape(arr, [arr.size])

    def tensor_with_shape(self, data, shape: Sequence[int]) -> SessionTensor:
        """session/mod.rs:180-198: InvalidShape(shape, [len]) when the data
        length is not the product of `shape`."""
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32).reshape(-1))
        shape = [int(s) for s in shape]
        if arr.size != _numel(shape):
            raise InvalidShape(shape, [arr.size])
        buf = _Buffer(self.device, arr.nbytes)
        if arr.nbytes:
            self.device.upload(buf.ptr, arr)
        return self._register(buf, shape)

    def import_(self, tensor: Tensor) -> SessionTensor:
        """session/mod.rs:204-207 `import`: copy an existing Tensor in.  The
        copy stays in HBM (device-to-device) instead of the reference's
        read-back and re-upload; the result is the same."""
        shape = tensor.shape()
        if tensor.device() is not self.device:
            return self.tensor_with_shape(tensor.to_vec(), shape)
        buf = _Buffer(self.device, 4 * _numel(shape))
        if buf.nbytes:
            dev = self.device
            with dev._lock:
                dev.check(dev._lib.bch_copy(dev.ctx, C.c_void_p(buf.ptr), C.c_void_p(tensor.ptr), buf.nbytes),
                          "import")
        return self._register(buf, shape)

    # -- ops ---------------------------------------------------------------
    def _same_shape(self, a: SessionTensor, b: SessionTensor) -> None:
        """session/mod.rs:571-580 check_same_shape."""
        if a._shape != b._shape:
            raise ShapeMismatch(a._shape, b._shape)

    def _elementwise(self, kind: str, *ins: SessionTensor, scalar: float = 0.0) -> SessionTensor:
        self._own(*ins)
        for t in ins[1:]:
            self._same_shape(ins[0], t)
        out = self._alloc_output(ins[0]._shape)
        ids = [t.buffer_id for t in ins] + [None] * (3 - len(ins))
        self._ops.append(("elementwise", kind, *ids, out.buffer_id, float(np.float32(scalar)), ins[0].len()))
        return out

    def add(self, a: SessionTensor, b: SessionTensor) -> SessionTensor:
        """a + b element-wise (session/mod.rs:214-226)."""
        return self._elementwise("add", a, b)

    def sub(self, a: SessionTensor, b: SessionTensor) -> SessionTensor:
        """a - b element-wise (session/mod.rs:228-240)."""
        return self._elementwise("sub", a, b)

    def mul(self, a: SessionTensor, b: SessionTensor) -> SessionTensor:
        """a * b element-wise (session/mod.rs:242-254)."""
        return self._elementwise("mul", a, b)

    def negate(self, a: SessionTensor) -> SessionTensor:
        """-a (session/mod.rs:256-264)."""
        return self._elementwise("negate", a)

    def fma(self, a: SessionTensor, b: SessionTensor, c: SessionTensor) -> SessionTensor:
        """fma(a, b, c) element-wise; a, b and c share one shape (session/mod.rs:268-287)."""
        return self._elementwise("fma", a, b, c)

    def scale(self, a: SessionTensor, scalar: float) -> SessionTensor:
        """a * scalar, the scalar as f32 (session/mod.rs:289-300)."""
        return self._elementwise("scale", a, scalar=scalar)

    def relu(self, a: SessionTensor) -> SessionTensor:
        """max(0, a) (session/mod.rs:340-347)."""
        return self._elementwise("relu", a)

    def gelu(self, a: SessionTensor) -> SessionTensor:
        """Tanh-form GELU, gelu_f64.wgsl (session/mod.rs:352-359)."""
        return self._elementwise("gelu", a)

    def layer_norm(self, a: SessionTensor, feature_size: int) -> SessionTensor:
        """Layer norm over consecutive groups of `feature_size` elements
        (session/mod.rs:379-398): InvalidInput when the element count is not
        a multiple of feature_size; epsilon 1e-5."""
        self._own(a)
        total = a.len()
        feature_size = int(feature_size)
        if feature_size == 0 or total % feature_size:
            raise InvalidInput(f"layer_norm: total {total} not divisible by feature_size {feature_size}")
        _usize_as_u32(feature_size)
        out = self._alloc_output(a._shape)
        self._ops.append(("layer_norm", a.buffer_id, out.buffer_id, total // feature_size, feature_size))
        return out

    def reshape(self, a: SessionTensor, new_shape: Sequence[int]) -> SessionTensor:
        """Metadata only: the same buffer with a new shape of the same element
        count, ShapeMismatch(new, old) otherwise (session/mod.rs:403-415)."""
        self._own(a)
        new_shape = [int(x) for x in new_shape]
        if _numel(new_shape) != a.len():
            raise ShapeMismatch(new_shape, a._shape)
        return SessionTensor(self, a.buffer_id, new_shape)

    def head_split(self, a: SessionTensor, dims: AttentionDims) -> SessionTensor:
        """[B, S, H*D] -> [B, H, S, D] for multi-head attention (session/mod.rs:423-446):
        InvalidInput when a's length is not B*S*H*D."""
        return self._head_permute("head_split", a, dims, "B×S×H×D",
                                  [dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim])

    def head_concat(self, a: SessionTensor, dims: AttentionDims) -> SessionTensor:
        """[B, H, S, D] -> [B, S, H*D] after multi-head attention (session/mod.rs:451-480):
        InvalidInput when a's length is not B*H*S*D."""
        return self._head_permute("head_concat", a, dims, "B×H×S×D",
                                  [dims.batch_size, dims.seq_len, dims.n_heads * dims.head_dim])

    def _head_permute(self, kind: str, a: SessionTensor, dims: AttentionDims, what: str,
                      out_shape: list[int]) -> SessionTensor:
        self._own(a)
        expected = dims.total_elements()
        if a.len() != expected:
            raise InvalidInput(f"{kind}: input len {a.len()} ≠ {what}={expected}")
        dims.as_u32()
        _check_i32(kind, self.device, batch=dims.batch_size, heads=dims.n_heads, seq=dims.seq_len,
                   head_dim=dims.head_dim, seq_x_head_dim=dims.seq_len * dims.head_dim,
                   heads_x_head_dim=dims.n_heads * dims.head_dim)
        out = self._alloc_output(out_shape)
        self._ops.append((kind, a.buffer_id, out.buffer_id, dims.batch_size, dims.seq_len, dims.n_heads,
                          dims.head_dim))
        return out

    # -- ops ---------------------------------------------------------------
    def matmul(self, a: SessionTensor, b: SessionTensor) -> SessionTensor:
        """output[m x n] = a[m x k] b[k x n] (session/mod.rs:305-333)."""
        self._own(a, b)
        if len(a._shape) != 2 or len(b._shape) != 2:
            raise InvalidShape(a._shape, b._shape)
        m, k = a._shape
        if b._shape[0] != k:
            raise ShapeMismatch([m, k], b._shape)
        n = b._shape[1]
        for v in (m, k, n):
            _usize_as_u32(v)
        _check_i32("matmul", self.device, m=m, n=n, k=k)
        out = self._alloc_output([m, n])
        self._ops.append(("matmul", a.buffer_id, b.buffer_id, out.buffer_id, m, k, n))
        return out

    def softmax(self, a: SessionTensor) -> SessionTensor:
        """exp(x - max) / sum over every element of `a` (session/mod.rs:364-371
        with the element count the reference passes as the shader's size,
        dispatch.rs:211)."""
        self._own(a)
        out = self._alloc_output(a._shape)
        self._ops.append(("softmax", a.buffer_id, out.buffer_id, a.len()))
        return out

    def attention(self, q: SessionTensor, k: SessionTensor, v: SessionTensor,
                  dims: AttentionDims) -> SessionTensor:
        """softmax(Q K^T / sqrt(D)) V over [B, H, S, D] (session/mod.rs:481-518)."""
        self._own(q, k, v)
        expected = dims.total_elements()
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.len() != expected:
                raise InvalidInput(f"attention: {name} len {t.len()} ≠ B×H×S×D={expected}")
        dims.as_u32()
        _check_i32("attention", self.device, batch=dims.batch_size, heads=dims.n_heads, seq=dims.seq_len,
                   head_dim=dims.head_dim)
        out = self._alloc_output([dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim])
        self._ops.append(("attention", q.buffer_id, k.buffer_id, v.buffer_id, out.buffer_id,
                          dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim))
        return out

    # -- execution ---------------------------------------------------------
    def run(self) -> None:
        """Enqueue every recorded op on the stream, in order, then wait once
        (session/mod.rs:521-540).  A launch error stops the batch and raises;
        ops enqueued before it have still been submitted."""
        if not self._ops:
            return
        dev = self.device
        lib, ctx = dev._lib, dev.ctx
        ptr = [C.c_void_p(b.ptr) for b in self._buffers]
        with dev._lock:
            for op in self._ops:
                kind = op[0]
                if kind == "matmul":
                    _, a, b, o, m, k, n = op
                    if m and n:
                        dev.check(lib.bch_sgemm(ctx, m, n, k, ptr[a], max(k, 1), ptr[b], max(n, 1), ptr[o],
                                                max(n, 1)), "matmul")
                elif kind == "elementwise":
                    _, name, a, b, c, o, scalar, n = op
                    if n:
                        code = _ELEMENTWISE[name][0]
                        pb = ptr[b] if b is not None else None
                        pc = ptr[c] if c is not None else None
                        dev.check(lib.bch_elementwise(ctx, code, n, ptr[a], pb, pc, scalar, ptr[o]), name)
                elif kind == "layer_norm":
                    _, a, o, rows, cols = op
                    if rows * cols:
                        dev.check(lib.bch_layer_norm(ctx, rows, cols, LAYER_NORM_EPS, ptr[a], ptr[o]),
                                  "layer_norm")
                elif kind == "softmax":
                    _, a, o, size = op
                    if size:
                        dev.check(lib.bch_softmax_rows(ctx, 1, size, ptr[a], ptr[o]), "softmax")
                elif kind == "attention":
                    _, q, k, v, o, b, h, s, d = op
                    if b * h * s * d:
                        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
                        dev.check(lib.bch_sdpa_fwd(ctx, b, h, s, s, d, scale, 0, ptr[q], ptr[k], ptr[v],
                                                   ptr[o]), "attention")
                elif kind in ("head_split", "head_concat"):
                    _, a, o, b, s, h, d = op
                    if b * s * h * d:
                        fn = lib.bch_head_split if kind == "head_split" else lib.bch_head_concat
                        dev.check(fn(ctx, b, s, h, d, ptr[a], ptr[o]), kind)
                else:  # pragma: no cover - ops are only appended above
                    raise ExecutionError(f"unknown session op {kind}")
            dev.check(lib.bch_sync(ctx), "run")
        self.executed = True

    # -- helpers -------------------------------------------------------------
    def _register(self, buf: _Buffer, shape: list[int]) -> SessionTensor:
        self._buffers.append(buf)
        self._shapes.append(list(shape))
        return SessionTensor(self, len(self._buffers) - 1, shape)

    def _alloc_output(self, shape: list[int]) -> SessionTensor:
        buf = _Buffer(self.device, 4 * _numel(shape))
        if buf.nbytes:
            dev = self.device
            with dev._lock:
                dev.check(dev._lib.bch_memset(dev.ctx, C.c_void_p(buf.ptr), 0, buf.nbytes), "alloc_output")
        return self._register(buf, shape)

    def _own(self, *ts: SessionTensor) -> None:
        for t in ts:
            if t._session is not self:
                raise InvalidInput("session tensor belongs to another TensorSession")


setattr(TensorSession, "import", TensorSession.import_)
