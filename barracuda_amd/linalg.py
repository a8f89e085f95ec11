"""f64 dense matrix multiply over the FP64 matrix cores (bch_dgemm), and the
f64 attention of the ml.attention handler.

Mirrors crates/barracuda/src/ops/linalg/gemm_f64.rs:
  GemmF64::{execute, execute_gemm, execute_gemm_ex}   gemm_f64.rs:77-249
  GemmCachedF64::{new, multiply, execute_to_buffer}   gemm_f64.rs:252-456
Host slices in, host vectors out, as in the reference (execute_to_buffer
returns the device buffer).  Same validation and messages.

attention_f64 is the computation of crates/barracuda-core/src/ipc/methods/
ml/forward.rs:121-150 (softmax(Q K^T / sqrt(d_k)) V in f64) on bch_dgemm and
bch_softmax_rows_f64; softmax_rows_f64 is its row softmax alone.

GemmCachedF64 in the reference dispatches (ceil(m/16), ceil(n/16)) workgroups
to a shader that reads x as the column (n) index (gemm_f64.rs:424-427 vs
gemm_f64.wgsl:31-32), so m != n leaves part of C unwritten; here every
element is computed.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .error import InvalidInput
from .tensor import HipDevice, _Buffer, _check_i32

__all__ = ["F64Buffer", "GemmCachedF64", "GemmF64", "attention_f64", "softmax_rows_f64"]


class F64Buffer:
    """A device buffer of f64 values (the wgpu::Buffer execute_to_buffer returns)."""

    def __init__(self, device: HipDevice, n: int):
        self.device = device
        self.len = int(n)
        self._buf = _Buffer(device, 8 * self.len)

    @property
    def ptr(self) -> int:
        return self._buf.ptr

    def upload(self, data) -> "F64Buffer":
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float64).reshape(-1))
        assert arr.size == self.len
        if arr.nbytes:
            self.device.upload(self.ptr, arr)
        return self

    def to_vec(self) -> np.ndarray:
        if self.len == 0:
            return np.empty(0, dtype=np.float64)
        return self.device.download(self.ptr, 8 * self.len).view(np.float64).copy()


def _dgemm(dev: HipDevice, a: F64Buffer, b: F64Buffer, c: F64Buffer, m: int, k: int, n: int, batch: int,
           alpha: float, beta: float, trans_a: bool, trans_b: bool) -> None:
    _check_i32("gemm_f64", dev, batch=batch, m=m, n=n, k=k)
    if batch * m * n == 0:
        return
    lda = max(m if trans_a else k, 1)
    ldb = max(k if trans_b else n, 1)
    with dev._lock:
        dev.check(dev._lib.bch_dgemm(dev.ctx, int(trans_a), int(trans_b), batch, m, n, k, float(alpha),
                                     C.c_void_p(a.ptr), lda, m * k, C.c_void_p(b.ptr), ldb, k * n, float(beta),
                                     C.c_void_p(c.ptr), max(n, 1), m * n), "gemm_f64")


class GemmF64:
    """gemm_f64.rs:77-249: batched C = alpha op(A) op(B) + beta C, packed row-major f64."""

    @staticmethod
    def execute(device: HipDevice, a, b, m: int, k: int, n: int, batch_size: int) -> np.ndarray:
        return GemmF64.execute_gemm(device, a, b, m, k, n, batch_size, 1.0, 0.0)

    @staticmethod
    def execute_gemm(device: HipDevice, a, b, m: int, k: int, n: int, batch_size: int, alpha: float,
                     beta: float) -> np.ndarray:
        return GemmF64.execute_gemm_ex(device, a, b, m, k, n, batch_size, alpha, beta, False, False)

    @staticmethod
    def execute_gemm_ex(device: HipDevice, a, b, m: int, k: int, n: int, batch_size: int, alpha: float,
                        beta: float, trans_a: bool, trans_b: bool) -> np.ndarray:
        a = np.asarray(a, dtype=np.float64).reshape(-1)
        b = np.asarray(b, dtype=np.float64).reshape(-1)
        expected_a, expected_b = batch_size * m * k, batch_size * k * n
        if a.size != expected_a:
            raise InvalidInput(f"A: expected {expected_a} elements, got {a.size}")
        if b.size != expected_b:
            raise InvalidInput(f"B: expected {expected_b} elements, got {b.size}")
        da = F64Buffer(device, a.size).upload(a)
        db = F64Buffer(device, b.size).upload(b)
        # the reference's C buffer is a fresh (zeroed) wgpu buffer: beta * C adds beta * 0
        dc = F64Buffer(device, batch_size * m * n).upload(np.zeros(batch_size * m * n))
        _dgemm(device, da, db, dc, m, k, n, batch_size, alpha, beta, trans_a, trans_b)
        return dc.to_vec()


class GemmCachedF64:
    """gemm_f64.rs:252-456: B uploaded once (a weight matrix), then C = A B for many A."""

    def __init__(self, device: HipDevice, b, k: int, n: int, batch_size: int):
        b = np.asarray(b, dtype=np.float64).reshape(-1)
        if b.size != batch_size * k * n:
            raise InvalidInput(f"GemmCachedF64: B has {b.size} elements, expected batch×K×N={batch_size * k * n}")
        self.device = device
        self.k, self.n, self.batch_size = k, n, batch_size
        self._b = F64Buffer(device, b.size).upload(b)

    @classmethod
    def new(cls, device: HipDevice, b, k: int, n: int, batch_size: int) -> "GemmCachedF64":
        return cls(device, b, k, n, batch_size)

    def multiply(self, a, m: int) -> np.ndarray:
        return self.execute_to_buffer(a, m).to_vec()

    def execute_to_buffer(self, a, m: int) -> F64Buffer:
        a = np.asarray(a, dtype=np.float64).reshape(-1)
        expected = self.batch_size * m * self.k
        if a.size != expected:
            raise InvalidInput(f"GemmCachedF64::execute_to_buffer: A has {a.size} elements, "
                               f"expected batch×M×K={expected}")
        da = F64Buffer(self.device, a.size).upload(a)
        dc = F64Buffer(self.device, self.batch_size * m * self.n)
        _dgemm(self.device, da, self._b, dc, m, self.k, self.n, self.batch_size, 1.0, 0.0, False, False)
        return dc


def _softmax_rows_f64(dev: HipDevice, x: F64Buffer, y: F64Buffer, rows: int, cols: int) -> None:
    with dev._lock:
        dev.check(dev._lib.bch_softmax_rows_f64(dev.ctx, rows, cols, C.c_void_p(x.ptr), C.c_void_p(y.ptr)),
                  "softmax_f64")


def softmax_rows_f64(device: HipDevice, x) -> np.ndarray:
    """The row softmax of ml.attention (ml/forward.rs:130-140) over the last
    axis of a float64 array: exp(x - max) / sum, the max skipping NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
    if x.ndim == 0 or x.size == 0:
        raise InvalidInput(f"softmax_rows_f64: empty input of shape {list(x.shape)}")
    cols = x.shape[-1]
    rows = x.size // cols
    buf = F64Buffer(device, x.size).upload(x)
    _softmax_rows_f64(device, buf, buf, rows, cols)
    return buf.to_vec().reshape(x.shape)


def attention_f64(device: HipDevice, q, k, v) -> np.ndarray:
    """ml/forward.rs:121-150 on the device, for row-major q [seq_q, d_k],
    k [seq_k, d_k], v [seq_k, d_v] (all non-empty, d_k >= 1):
      scores = (Q K^T) * (1 / sqrt(d_k))     bch_dgemm, B transposed, alpha
      P      = row softmax of scores         bch_softmax_rows_f64, in place
      out    = P V                           bch_dgemm
    Returns [seq_q, d_v] float64."""
    q, k, v = (np.ascontiguousarray(np.asarray(a, dtype=np.float64)) for a in (q, k, v))
    (sq, dk), (sk, dk2), (sk2, dv) = q.shape, k.shape, v.shape
    if sq < 1 or sk < 1 or dk < 1 or dk2 != dk or sk2 != sk:
        raise InvalidInput(f"attention_f64: q {list(q.shape)}, k {list(k.shape)}, v {list(v.shape)}")
    if dv == 0:
        return np.zeros((sq, 0), dtype=np.float64)
    dq, dkb, dvb = (F64Buffer(device, a.size).upload(a) for a in (q, k, v))
    scores = F64Buffer(device, sq * sk)
    out = F64Buffer(device, sq * dv)
    scale = 1.0 / float(np.sqrt(np.float64(dk)))
    _dgemm(device, dq, dkb, scores, sq, dk, sk, 1, scale, 0.0, False, True)
    _softmax_rows_f64(device, scores, scores, sq, sk)
    _dgemm(device, scores, dvb, out, sq, sk, dv, 1, 1.0, 0.0, False, False)
    return out.to_vec().reshape(sq, dv)
