"""Host side of the hot path: barraCuda's op API over libbarracuda_hip.so.

Mirrors the reference's Rust surface for this path (same method names,
argument meaning and error variants), with every computation routed through
the C ABI to the gfx950 kernels.  There is no CPU fallback: if the library
or the device is missing, the call raises.

Reference (crates/barracuda/src/):
  Tensor::{from_data, shape, to_vec}            tensor/mod.rs:185, 409, 448
  Tensor::matmul / matmul_ref, MatMul            ops/matmul.rs:49-243
  Tensor::matmul_tiled, MatmulTiled              ops/matmul_tiled.rs:45-171
  Tensor::batch_matmul, BatchMatMul              ops/batch_matmul.rs:24-163
  Tensor::softmax, Softmax (global)              ops/softmax.rs:31-144
  Tensor::softmax_dim                            ops/tensor_axis_ops.rs:67-126
  Tensor::attention, Attention                   ops/attention/mod.rs:84-206
  Tensor::scaled_dot_product_attention           ops/scaled_dot_product_attention/mod.rs:81-226
  Tensor::causal_attention, CausalAttention      ops/causal_attn/mod.rs:64-158
  FlashAttention                                 ops/flash_attention.rs:45-146
  Tensor::grouped_query_attention                ops/grouped_query_attention/mod.rs:52-226
  Tensor::multi_head_attention                   ops/mha/mod.rs:48-263, projections.rs:18-58
  Tensor::reshape                                tensor/mod.rs (shape-only view)
"""
from __future__ import annotations

import ctypes as C
import math
import threading
from pathlib import Path
from typing import Sequence

import numpy as np

from . import _native as N
from .error import (BarracudaError, DeviceError, DeviceNotAvailable, InvalidInput,
                    InvalidOperation, ShapeMismatch, UnsupportedOperation, from_status)

__all__ = [
    "HipDevice", "get_device", "Tensor", "MatMul", "MatmulTiled", "BatchMatMul",
    "Softmax", "Attention", "ScaledDotProductAttention", "CausalAttention",
    "FlashAttention", "GroupedQueryAttention", "MultiHeadAttention", "LcgStream",
    "ReLU", "GELU", "LayerNorm",
]


class HipDevice:
    """One bch_ctx (device + stream).  Plays the role of the reference's
    WgpuDevice behind GpuBackend (device/backend.rs:244-444).  Calls are
    serialised with a lock: a context is not re-entrant."""

    def __init__(self, device: int = -1, code_object_dir: str | None = None):
        self._lib = N.load()
        self._lock = threading.RLock()
        ctx = C.c_void_p()
        st = self._lib.bch_ctx_create(device, code_object_dir.encode() if code_object_dir else None,
                                      C.byref(ctx))
        if st != N.BCH_OK:
            raise from_status(st, N.last_error(None), "device")
        self._ctx = ctx
        self.ordinal = device

    # -- plumbing --------------------------------------------------------
    @property
    def ctx(self) -> C.c_void_p:
        return self._ctx

    def name(self) -> str:
        return "hip:gfx950"

    def is_lost(self) -> bool:
        """GpuBackend::is_lost (device/backend.rs:256): whether a call on this
        context has reported a lost device (a kernel fault, an uncorrectable
        ECC error).  Sticky: every later device call raises DeviceLost."""
        flag = C.c_int(0)
        with self._lock:
            self.check(self._lib.bch_ctx_is_lost(self._ctx, C.byref(flag)), "is_lost")
        return bool(flag.value)

    def check(self, status: int, op: str) -> None:
        if status != N.BCH_OK:
            raise from_status(status, N.last_error(self._ctx), op, self.name())

    def alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        with self._lock:
            self.check(self._lib.bch_alloc(self._ctx, nbytes, C.byref(p)), "alloc_buffer")
        return p.value or 0

    def free(self, ptr: int) -> None:
        if ptr and self._ctx:
            with self._lock:
                self.check(self._lib.bch_free(self._ctx, C.c_void_p(ptr)), "free")

    def upload(self, ptr: int, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host)
        with self._lock:
            self.check(self._lib.bch_upload(self._ctx, C.c_void_p(ptr), host.ctypes.data_as(C.c_void_p),
                                            host.nbytes), "upload")

    def download(self, ptr: int, nbytes: int) -> np.ndarray:
        out = np.empty(nbytes // 4, dtype=np.float32)
        with self._lock:
            self.check(self._lib.bch_download(self._ctx, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr),
                                              nbytes), "download")
        return out

    def sync(self) -> None:
        with self._lock:
            self.check(self._lib.bch_sync(self._ctx), "sync")

    def dispatch_binary(self, binary: bytes | str | Path, entry: str, workgroups: Sequence[int],
                        block: Sequence[int], args: Sequence[C._SimpleCData],
                        shared_bytes: int = 0) -> None:
        """GpuBackend::dispatch_binary (device/backend.rs:344-354): launch a
        precompiled gfx950 code object.  `binary` is the image bytes or a
        path; `args` are ctypes scalars / c_void_p in kernel-argument order."""
        grid = (C.c_uint * 3)(*workgroups)
        blk = (C.c_uint * 3)(*block)
        argv = (C.c_void_p * max(1, len(args)))(*[C.cast(C.pointer(a), C.c_void_p) for a in args])
        if isinstance(binary, (str, Path)):
            img = C.c_char_p(str(binary).encode())
            length = 0
        else:
            img = C.create_string_buffer(bytes(binary), len(binary))
            length = len(binary)
        with self._lock:
            self.check(self._lib.bch_launch_code_object(self._ctx, C.cast(img, C.c_void_p), length,
                                                        entry.encode(), grid, blk, argv, len(args),
                                                        shared_bytes), "dispatch_binary")

    def close(self) -> None:
        if self._ctx:
            with self._lock:
                self._lib.bch_ctx_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default: HipDevice | None = None
_default_lock = threading.Lock()


def get_device() -> HipDevice:
    """The process-wide default device (BARRACUDA_HIP_DEVICE or 0)."""
    global _default
    with _default_lock:
        if _default is None:
            _default = HipDevice(-1)
        return _default


class _Buffer:
    """Owned device allocation (RAII free), shared between Tensor clones."""

    __slots__ = ("device", "ptr", "nbytes", "__weakref__")

    def __init__(self, device: HipDevice, nbytes: int):
        self.device = device
        self.nbytes = nbytes
        self.ptr = device.alloc(nbytes) if nbytes else 0

    def __del__(self):
        try:
            if self.ptr:
                self.device.free(self.ptr)
        except Exception:
            pass


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


class Tensor:
    """f32 tensor resident in HBM (tensor/mod.rs:47-60, with a HIP buffer)."""

    def __init__(self, buffer: _Buffer, shape: Sequence[int], device: HipDevice):
        self._buf = buffer
        self._shape = [int(s) for s in shape]
        self._device = device

    # -- construction / readback ------------------------------------------
    @classmethod
    def from_data(cls, data, shape: Sequence[int], device: HipDevice | None = None) -> "Tensor":
        """tensor/mod.rs:185 from_data: upload f32 data with a shape."""
        device = device or get_device()
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32).reshape(-1))
        if arr.size != _numel(shape):
            raise ShapeMismatch([_numel(shape)], [arr.size])
        buf = _Buffer(device, arr.nbytes)
        if arr.nbytes:
            device.upload(buf.ptr, arr)
        return cls(buf, shape, device)

    from_vec_on = from_data

    @classmethod
    def empty(cls, shape: Sequence[int], device: HipDevice | None = None) -> "Tensor":
        device = device or get_device()
        return cls(_Buffer(device, 4 * _numel(shape)), shape, device)

    def shape(self) -> list[int]:
        return list(self._shape)

    def len(self) -> int:
        return _numel(self._shape)

    def device(self) -> HipDevice:
        return self._device

    @property
    def ptr(self) -> int:
        return self._buf.ptr

    def to_vec(self) -> np.ndarray:
        """tensor/mod.rs:448 to_vec: blocking readback, flat f32."""
        if self._buf.nbytes == 0:
            return np.empty(0, dtype=np.float32)
        return self._device.download(self._buf.ptr, self._buf.nbytes)

    def to_numpy(self) -> np.ndarray:
        return self.to_vec().reshape(self._shape)

    def clone(self) -> "Tensor":
        """Shares the buffer, as Tensor::clone bumps a refcount (tensor/mod.rs:267-278)."""
        return Tensor(self._buf, self._shape, self._device)

    def reshape(self, shape: Sequence[int]) -> "Tensor":
        """Same buffer, new shape with the same element count (the reference's
        reshape, used by MultiHeadAttention at ops/mha/projections.rs:32-35)."""
        shape = [int(x) for x in shape]
        if _numel(shape) != self.len():
            raise ShapeMismatch(shape, self._shape)
        return Tensor(self._buf, shape, self._device)

    # -- ops (same names as the reference) -----------------------------------
    def matmul(self, other: "Tensor") -> "Tensor":
        return MatMul(self, other).execute()

    def matmul_ref(self, other: "Tensor") -> "Tensor":
        return MatMul(self, other).execute()

    def matmul_tiled(self, other: "Tensor") -> "Tensor":
        return MatmulTiled(self, other).execute()

    def batch_matmul(self, other: "Tensor") -> "Tensor":
        return BatchMatMul(self, other).execute()

    def softmax(self) -> "Tensor":
        return Softmax(self).execute()

    def softmax_dim(self, axis: int) -> "Tensor":
        """ops/tensor_axis_ops.rs:67-126: softmax along `axis`."""
        shape = self._shape
        if not shape:
            raise InvalidOperation("softmax_dim", "Empty tensor not supported")
        if axis >= len(shape) or axis < 0:
            raise InvalidOperation("softmax_dim", f"Axis {axis} out of bounds for shape {shape}")
        out = Tensor.empty(shape, self._device)
        outer = _numel(shape[:axis])
        inner = _numel(shape[axis + 1:])
        if outer * shape[axis] * inner == 0:
            return out
        dev = self._device
        with dev._lock:
            dev.check(dev._lib.bch_softmax_axis(dev.ctx, outer, shape[axis], inner,
                                                C.c_void_p(self.ptr), C.c_void_p(out.ptr)),
                      "softmax_dim")
        return out

    def relu(self) -> "Tensor":
        """ops/relu.rs:106: max(x, 0) element-wise."""
        return ReLU(self).execute()

    def gelu_wgsl(self) -> "Tensor":
        """ops/gelu_wgsl.rs:147: tanh-form GELU element-wise."""
        return GELU(self).execute()

    def layer_norm_wgsl(self, epsilon: float) -> "Tensor":
        """ops/layer_norm_wgsl.rs:160-165: layer norm over the last axis."""
        return LayerNorm(self, epsilon).execute()

    def attention(self, key: "Tensor", value: "Tensor") -> "Tensor":
        return Attention(self, key, value).execute()

    def scaled_dot_product_attention(self, key: "Tensor", value: "Tensor") -> "Tensor":
        return ScaledDotProductAttention(self, key, value).execute()

    def causal_attention(self, key: "Tensor", value: "Tensor") -> "Tensor":
        return CausalAttention(self, key, value).execute()

    def grouped_query_attention(self, key: "Tensor", value: "Tensor") -> "Tensor":
        return GroupedQueryAttention(self, key, value).execute()

    def multi_head_attention(self, key: "Tensor", value: "Tensor", w_q: "Tensor", w_k: "Tensor",
                             w_v: "Tensor", w_o: "Tensor", num_heads: int) -> "Tensor":
        return MultiHeadAttention(self, key, value, w_q, w_k, w_v, w_o, num_heads).execute()


class LcgStream:
    """Seeded input stream over the reference's generators, filled in HBM
    (bch_fill_uniform / bch_fill_normal).  Successive tensors continue one
    stream, as the reference fills arrays in argument order: uniform is
    rng.rs:20-70, normal is ops/lattice/constants.rs:38-49 (Box-Muller)."""

    def __init__(self, seed: int, device: HipDevice | None = None):
        self.state = C.c_ulonglong(seed)
        self.device = device or get_device()

    def uniform(self, shape: Sequence[int], lo: float = -1.0, hi: float = 1.0) -> Tensor:
        t = Tensor.empty(shape, self.device)
        dev = self.device
        with dev._lock:
            dev.check(dev._lib.bch_fill_uniform(dev.ctx, C.c_void_p(t.ptr), t.len(), C.byref(self.state),
                                                lo, hi), "fill_uniform")
        return t

    def normal(self, shape: Sequence[int], mu: float = 0.0, sigma: float = 1.0) -> Tensor:
        t = Tensor.empty(shape, self.device)
        dev = self.device
        with dev._lock:
            dev.check(dev._lib.bch_fill_normal(dev.ctx, C.c_void_p(t.ptr), t.len(), C.byref(self.state),
                                               mu, sigma), "fill_normal")
        return t


def _same_device(*ts: Tensor) -> HipDevice:
    dev = ts[0].device()
    for t in ts[1:]:
        if t.device() is not dev:
            raise DeviceError("tensors live on different devices")
    return dev


_I32_MAX = 2**31 - 1


def _check_i32(op: str, dev: HipDevice, **dims: int) -> None:
    """The C ABI takes GEMM / attention dimensions as int; ctypes would wrap a
    larger value silently, so refuse it here."""
    for name, v in dims.items():
        if v > _I32_MAX:
            raise UnsupportedOperation(op, f"{dev.name()} ({name}={v} exceeds 2^31-1)")


def _sgemm(dev: HipDevice, m: int, n: int, k: int, a: Tensor, b: Tensor, op: str) -> Tensor:
    _check_i32(op, dev, m=m, n=n, k=k)
    out = Tensor.empty([m, n], dev)
    if m * n == 0:
        return out
    with dev._lock:
        dev.check(dev._lib.bch_sgemm(dev.ctx, m, n, k, C.c_void_p(a.ptr), max(k, 1), C.c_void_p(b.ptr),
                                     max(n, 1), C.c_void_p(out.ptr), max(n, 1)), op)
    return out


class MatMul:
    """ops/matmul.rs:49-214: C[m,n] = A[m,k] B[k,n]."""

    def __init__(self, lhs: Tensor, rhs: Tensor):
        self.lhs, self.rhs = lhs, rhs

    def execute(self) -> Tensor:
        ls, rs = self.lhs.shape(), self.rhs.shape()
        if len(ls) < 2 or len(rs) < 2:
            raise InvalidOperation("matmul", f"requires 2D+ tensors, got shapes {ls} and {rs}")
        # >= 3-D inputs use shape[0], shape[1] (matmul.rs:103-107)
        m, k = ls[0], ls[1]
        k_rhs, n = rs[0], rs[1]
        if k != k_rhs:
            raise ShapeMismatch(ls, rs)
        dev = _same_device(self.lhs, self.rhs)
        return _sgemm(dev, m, n, k, self.lhs, self.rhs, "matmul")


class MatmulTiled(MatMul):
    """ops/matmul_tiled.rs:45-122: same contract as MatMul."""


class BatchMatMul:
    """ops/batch_matmul.rs:24-144: A[batch,m,k] . B[batch,k,n] -> [batch,m,n].

    The reference reads batch/m/k from A and n from B without checking that
    B agrees; here a disagreeing B is a ShapeMismatch instead of reading out
    of bounds."""

    def __init__(self, a: Tensor, b: Tensor):
        self.a, self.b = a, b

    def execute(self) -> Tensor:
        as_, bs = self.a.shape(), self.b.shape()
        if len(as_) != 3 or len(bs) != 3:
            raise InvalidOperation("batch_matmul", f"requires 3D tensors, got shapes {as_} and {bs}")
        batch, m, k = as_
        if bs[0] != batch or bs[1] != k:
            raise ShapeMismatch(as_, bs)
        n = bs[2]
        dev = _same_device(self.a, self.b)
        _check_i32("batch_matmul", dev, batch=batch, m=m, n=n, k=k)
        out = Tensor.empty([batch, m, n], dev)
        if batch * m * n == 0:
            return out
        with dev._lock:
            dev.check(dev._lib.bch_sgemm_strided_batched(
                dev.ctx, batch, m, n, k, C.c_void_p(self.a.ptr), m * k, C.c_void_p(self.b.ptr), k * n,
                C.c_void_p(out.ptr), m * n), "batch_matmul")
        return out


class Softmax:
    """ops/softmax.rs:31-133: softmax over ALL elements of the tensor."""

    def __init__(self, t: Tensor):
        if not t.shape():
            raise InvalidOperation("Softmax", "Empty tensor not supported")
        self.t = t

    def execute(self) -> Tensor:
        dev = self.t.device()
        out = Tensor.empty(self.t.shape(), dev)
        size = self.t.len()
        if size == 0:
            return out
        with dev._lock:
            dev.check(dev._lib.bch_softmax_rows(dev.ctx, 1, size, C.c_void_p(self.t.ptr),
                                                C.c_void_p(out.ptr)), "softmax")
        return out


def _elementwise(dev: HipDevice, op: int, out: Tensor, a: Tensor, b: Tensor | None = None,
                 c: Tensor | None = None, scalar: float = 0.0, name: str = "elementwise") -> Tensor:
    n = out.len()
    if n:
        p = lambda t: C.c_void_p(t.ptr) if t is not None else None
        with dev._lock:
            dev.check(dev._lib.bch_elementwise(dev.ctx, op, n, p(a), p(b), p(c), float(scalar), p(out)), name)
    return out


class ReLU:
    """ops/relu.rs: max(x, 0) over every element (relu_f64.wgsl)."""

    def __init__(self, input: Tensor):
        self.input = input

    def execute(self) -> Tensor:
        dev = self.input.device()
        return _elementwise(dev, N.BCH_EW_RELU, Tensor.empty(self.input.shape(), dev), self.input, name="relu")


class GELU:
    """ops/gelu_wgsl.rs:33-141: x Phi(x) in the tanh form of gelu_f64.wgsl,
    0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))), over every element."""

    def __init__(self, input: Tensor):
        self.input = input

    def execute(self) -> Tensor:
        dev = self.input.device()
        return _elementwise(dev, N.BCH_EW_GELU, Tensor.empty(self.input.shape(), dev), self.input, name="gelu")


class LayerNorm:
    """ops/layer_norm_wgsl.rs:47-157: normalise each row along the last
    dimension, (x - mean) / sqrt(var + epsilon), biased variance, no affine
    parameters (layer_norm_f64.wgsl)."""

    def __init__(self, input: Tensor, epsilon: float):
        self.input = input
        self.epsilon = float(epsilon)

    def execute(self) -> Tensor:
        shape = self.input.shape()
        if not shape:
            raise InvalidOperation("LayerNorm", "Empty tensor not supported")
        dev = self.input.device()
        out = Tensor.empty(shape, dev)
        cols = shape[-1]
        rows = _numel(shape[:-1])
        if rows * cols:
            with dev._lock:
                dev.check(dev._lib.bch_layer_norm(dev.ctx, rows, cols, self.epsilon, C.c_void_p(self.input.ptr),
                                                  C.c_void_p(out.ptr)), "layer_norm")
        return out


def _sdpa(dev: HipDevice, q: Tensor, k: Tensor, v: Tensor, causal: bool, op: str,
          b: int, h: int, sq: int, skv: int, d: int) -> Tensor:
    _check_i32(op, dev, batch=b, heads=h, q_len=sq, kv_len=skv, head_dim=d)
    out = Tensor.empty(q.shape(), dev)
    if b * h * sq * d == 0:
        return out
    if skv == 0:
        raise InvalidOperation(op, "key sequence is empty (shape/dimension mismatch)")
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    with dev._lock:
        dev.check(dev._lib.bch_sdpa_fwd(dev.ctx, b, h, sq, skv, d, float(scale), int(causal),
                                        C.c_void_p(q.ptr), C.c_void_p(k.ptr), C.c_void_p(v.ptr),
                                        C.c_void_p(out.ptr)), op)
    return out


class Attention:
    """ops/attention/mod.rs:96-144 (validation) + compute.rs:21-111: softmax(QK^T/sqrt(D)) V,
    Q [B,H,Sq,D], K/V [B,H,Skv,D] (cross-attention allowed)."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor):
        for name, t in (("query", query), ("key", key), ("value", value)):
            if len(t.shape()) != 4:
                raise InvalidOperation(
                    "attention",
                    f"{name} requires 4D tensor [batch, heads, seq_len, head_dim], got {len(t.shape())}D")
        qs, ks, vs = query.shape(), key.shape(), value.shape()
        if qs[0] != ks[0] or qs[1] != ks[1] or qs[3] != ks[3]:
            raise ShapeMismatch(qs, ks)
        if ks != vs:
            raise ShapeMismatch(ks, vs)
        self.q, self.k, self.v = query, key, value

    def execute(self) -> Tensor:
        b, h, sq, d = self.q.shape()
        skv = self.k.shape()[2]
        dev = _same_device(self.q, self.k, self.v)
        return _sdpa(dev, self.q, self.k, self.v, False, "attention", b, h, sq, skv, d)


class ScaledDotProductAttention:
    """ops/scaled_dot_product_attention/mod.rs:101-149: self-attention, Q, K, V same shape."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor):
        qs, ks, vs = query.shape(), key.shape(), value.shape()
        if len(qs) != 4 or len(ks) != 4 or len(vs) != 4:
            raise InvalidInput("Q, K, V must be 4D tensors [batch, heads, seq_len, head_dim]")
        if ks != qs or vs != qs:
            raise ShapeMismatch(qs, vs if ks == qs else ks)
        _same_device(query, key, value)
        self.q, self.k, self.v = query, key, value

    def execute(self) -> Tensor:
        b, h, s, d = self.q.shape()
        return _sdpa(self.q.device(), self.q, self.k, self.v, False, "scaled_dot_product_attention",
                     b, h, s, s, d)


class CausalAttention:
    """ops/causal_attn/mod.rs:64-158: causal SDPA (key j <= query i), Q, K, V same shape.

    The reference's GPU dispatch computes only rows i < 16 of head 0
    (1-D grids for 2-D shaders, causal_attn/compute.rs:69-108); this
    follows its CPU definition (ops/causal_attention.rs:52-134) for every
    row and head."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor):
        qs, ks, vs = query.shape(), key.shape(), value.shape()
        if len(qs) != 4 or len(ks) != 4 or len(vs) != 4:
            raise ShapeMismatch(qs, ks)
        if qs != ks or qs != vs:
            raise ShapeMismatch(qs, ks)
        self.q, self.k, self.v = query, key, value

    def execute(self) -> Tensor:
        b, h, s, d = self.q.shape()
        dev = _same_device(self.q, self.k, self.v)
        return _sdpa(dev, self.q, self.k, self.v, True, "causal_attention", b, h, s, s, d)


class FlashAttention:
    """ops/flash_attention.rs:45-146: 2-D [seq_len, head_dim] single-head attention,
    scale 1/sqrt(head_dim).  The reference shader keeps at most 256 keys
    (flash_attention_f64.wgsl:70-71); here every key is attended to, so the
    two agree for seq_len <= 256."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor, num_heads: int = 1):
        if query.shape() != key.shape() or query.shape() != value.shape():
            raise InvalidOperation(
                "FlashAttention",
                f"Q, K, V must have same shape, got Q: {query.shape()}, K: {key.shape()}, V: {value.shape()}")
        if len(query.shape()) != 2:
            raise InvalidOperation("FlashAttention",
                                   f"Requires 2D tensors [seq_len, head_dim], got shape: {query.shape()}")
        self.q, self.k, self.v = query, key, value
        self.num_heads = num_heads

    def execute(self) -> Tensor:
        s, d = self.q.shape()
        dev = _same_device(self.q, self.k, self.v)
        return _sdpa(dev, self.q, self.k, self.v, False, "FlashAttention", 1, 1, s, s, d)


def _dense(h: int, s: int, d: int) -> N.AttnLayout:
    """[B, H, S, D] row-major."""
    return N.AttnLayout(h * s * d, s * d, d)


def _sdpa_ex(dev: HipDevice, op: str, b: int, h: int, hkv: int, sq: int, skv: int, d: int, causal: bool,
             q: Tensor, ql: N.AttnLayout, k: Tensor, kl: N.AttnLayout, v: Tensor, vl: N.AttnLayout,
             o: Tensor, ol: N.AttnLayout) -> None:
    """bch_sdpa_fwd_ex: strided operands, hkv key/value heads, scale 1/sqrt(d)."""
    _check_i32(op, dev, batch=b, heads=h, kv_heads=hkv, q_len=sq, kv_len=skv, head_dim=d)
    if b * h * sq * d == 0:
        return
    if skv == 0:
        raise InvalidOperation(op, "key sequence is empty (shape/dimension mismatch)")
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    with dev._lock:
        dev.check(dev._lib.bch_sdpa_fwd_ex(dev.ctx, b, h, hkv, sq, skv, d, float(scale), int(causal),
                                           C.c_void_p(q.ptr), ql, C.c_void_p(k.ptr), kl, C.c_void_p(v.ptr), vl,
                                           C.c_void_p(o.ptr), ol), op)


class GroupedQueryAttention:
    """ops/grouped_query_attention/mod.rs:52-147 (validation) + compute.rs:27-121:
    Q [B, Hq, S, D], K/V [B, Hkv, S, D], query head h attends with key/value
    head h / (Hq / Hkv); softmax(Q K^T / sqrt(D)) V, non-causal.  One fused
    launch replaces the reference's three passes and its two [B, Hq, S, S]
    intermediates."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor):
        qs, ks, vs = query.shape(), key.shape(), value.shape()
        if len(qs) != 4 or len(ks) != 4 or len(vs) != 4:
            raise InvalidInput("All inputs must be 4D tensors [batch, heads, seq_len, head_dim]")
        b, hq, s, d = qs
        if ks[0] != b or ks[2] != s or ks[3] != d:
            raise ShapeMismatch([b, hq, s, d], ks)
        if vs != ks:
            raise ShapeMismatch(ks, vs)
        hkv = ks[1]
        if hkv == 0 or hq % hkv != 0:
            raise InvalidInput(f"num_q_heads ({hq}) must be divisible by num_kv_heads ({hkv})")
        if query.device() is not key.device() or query.device() is not value.device():
            raise DeviceError("All tensors must be on the same device")
        self.q, self.k, self.v = query, key, value

    def execute(self) -> Tensor:
        b, hq, s, d = self.q.shape()
        hkv = self.k.shape()[1]
        dev = self.q.device()
        out = Tensor.empty([b, hq, s, d], dev)
        _sdpa_ex(dev, "grouped_query_attention", b, hq, hkv, s, s, d, False,
                 self.q, _dense(hq, s, d), self.k, _dense(hkv, s, d), self.v, _dense(hkv, s, d),
                 out, _dense(hq, s, d))
        return out


class MultiHeadAttention:
    """ops/mha/mod.rs:48-187 + projections.rs:18-58: query [B, Sq, D], key /
    value [B, Skv, D], weights [D, D]; heads = D / num_heads wide.

        Q' = query W_q, K' = key W_k, V' = value W_v      (three GEMMs)
        O[b, i, h] = attention(Q'[b, :, h], K'[b, :, h], V'[b, :, h])
        out = O W_o                                        (one GEMM)

    The reference copies each projection into [B, H, S, D/H] (head_split) and
    the attention output back into [B, S, D] (head_concat); here the fused
    attention reads the [B, S, H, D/H] projections and writes the [B, S, H,
    D/H] output through strides, so neither copy exists."""

    def __init__(self, query: Tensor, key: Tensor, value: Tensor, w_q: Tensor, w_k: Tensor, w_v: Tensor,
                 w_o: Tensor, num_heads: int):
        qs, ks, vs = query.shape(), key.shape(), value.shape()
        if len(qs) != 3 or len(ks) != 3 or len(vs) != 3:
            raise ShapeMismatch(qs, [0, 0, 0])
        if qs[0] != ks[0] or qs[0] != vs[0]:
            raise ShapeMismatch(qs, ks)
        if qs[2] != ks[2] or ks[2] != vs[2]:
            raise ShapeMismatch(qs, ks)
        if ks != vs:
            raise ShapeMismatch(ks, vs)
        ws = [w.shape() for w in (w_q, w_k, w_v, w_o)]
        if any(len(w) != 2 for w in ws):
            raise ShapeMismatch(ws[0], [0, 0])
        d = qs[2]
        if any(w != [d, d] for w in ws):
            raise ShapeMismatch(ws[0], [d, d])
        if num_heads == 0 or d % num_heads != 0:
            raise InvalidOperation("multi_head_attention",
                                   f"d_model ({d}) must be divisible by num_heads ({num_heads})")
        self.q, self.k, self.v = query, key, value
        self.w_q, self.w_k, self.w_v, self.w_o = w_q, w_k, w_v, w_o
        self.num_heads = num_heads

    def execute(self) -> Tensor:
        b, sq, d = self.q.shape()
        skv = self.k.shape()[1]
        h = self.num_heads
        hd = d // h
        dev = _same_device(self.q, self.k, self.v, self.w_q, self.w_k, self.w_v, self.w_o)
        qp = _sgemm(dev, b * sq, d, d, self.q, self.w_q, "multi_head_attention")
        kp = _sgemm(dev, b * skv, d, d, self.k, self.w_k, "multi_head_attention")
        vp = _sgemm(dev, b * skv, d, d, self.v, self.w_v, "multi_head_attention")
        o = Tensor.empty([b * sq, d], dev)
        # head h of row i of batch b is at b*S*d + i*d + h*hd: the [B, S, H, hd] view
        _sdpa_ex(dev, "multi_head_attention", b, h, h, sq, skv, hd, False,
                 qp, N.AttnLayout(sq * d, hd, d), kp, N.AttnLayout(skv * d, hd, d),
                 vp, N.AttnLayout(skv * d, hd, d), o, N.AttnLayout(sq * d, hd, d))
        return _sgemm(dev, b * sq, d, d, o, self.w_o, "multi_head_attention").reshape([b, sq, d])
