"""ctypes wrapper of oracle/libbc_oracle.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product (barracuda_amd/) never imports it.  See bc_oracle.c for what each
function restates (reference file:line) and how it is pinned.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("BC_ORACLE_LIB", HERE / "libbc_oracle.so"))

_lib = None
_fp = C.POINTER(C.c_float)
_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)
_u64p = C.POINTER(C.c_uint64)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        L.bco_lcg_advance.restype = C.c_uint64
        L.bco_lcg_advance.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.bco_fill_uniform.argtypes = [_u64p, C.c_double, C.c_double, _fp, C.c_size_t]
        L.bco_fill_normal.argtypes = [_u64p, C.c_double, C.c_double, _fp, C.c_size_t]
        L.bco_matmul_f64.argtypes = [C.c_int, C.c_int, C.c_int, _fp, C.c_long, _fp, C.c_long, _dp,
                                     C.c_long, _ip, C.c_int]
        L.bco_softmax_rows_f64.argtypes = [C.c_long, C.c_long, _fp, _dp]
        L.bco_sdpa_f64.argtypes = [C.c_int] * 5 + [C.c_double, C.c_int, _fp, _fp, _fp, _dp, _ip, C.c_int]
        L.bco_sdpa_f64_rows.argtypes = [C.c_int] * 5 + [C.c_double, C.c_int, _fp, _fp, _fp, _dp, _ip, C.c_int]
        L.bco_matmul_cpu_exec_f32.argtypes = [C.c_int, C.c_int, C.c_int, _fp, _fp, _fp, C.c_int, C.c_int]
        L.bco_matmul_k1_f32.argtypes = [C.c_int, C.c_int, C.c_int, _fp, _fp, _fp]
        L.bco_batch_matmul_seq_f32.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, _fp, _fp, _fp]
        L.bco_softmax_dim_f32.argtypes = [C.c_long, C.c_long, C.c_long, _fp, _fp, C.c_long, C.c_long]
        L.bco_softmax_global_f32.argtypes = [C.c_long, _fp, _fp]
        L.bco_attention_3pass_f32.argtypes = [C.c_int] * 6 + [_fp, _fp, _fp, _fp, _ip, C.c_int]
        L.bco_causal_attention_cpu_f32.argtypes = [C.c_int] * 4 + [_fp, _fp, _fp, _fp, C.c_int, C.c_int]
        L.bco_linear_f32.argtypes = [C.c_int] * 3 + [_fp, _fp, _fp, C.c_int, _fp]
        L.bco_gemm_f64_wgsl.argtypes = [C.c_int] * 6 + [C.c_double, _dp, _dp, C.c_double, _dp, _dp]
        L.bco_max_rel_err.restype = C.c_double
        L.bco_max_rel_err.argtypes = [C.c_size_t, _fp, _dp]
        L.bco_max_rel_err_f32ref.restype = C.c_double
        L.bco_max_rel_err_f32ref.argtypes = [C.c_size_t, _fp, _fp]
        L.bco_num_threads.restype = C.c_int
        L.bco_set_num_threads.argtypes = [C.c_int]
        L.bco_gelu_f64.argtypes = [C.c_size_t, _fp, _dp]
        L.bco_gelu_wgsl_f32.argtypes = [C.c_size_t, _fp, _fp]
        L.bco_layer_norm_f64.argtypes = [C.c_long, C.c_long, C.c_double, _fp, _dp]
        L.bco_layer_norm_f32.argtypes = [C.c_long, C.c_long, C.c_float, _fp, _fp]
        L.bco_ml_softmax_rows_f64.argtypes = [C.c_long, C.c_long, _dp, _dp]
        L.bco_ml_attention_f64.argtypes = [C.c_int] * 4 + [_dp, _dp, _dp, _dp]
        L.bco_matmul_inline_f64.argtypes = [C.c_int] * 3 + [_dp, _dp, _dp]
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _d(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(_dp)


def _sel(sel):
    if sel is None:
        return None, 0, None
    arr = np.ascontiguousarray(np.asarray(sel, dtype=np.int32))
    return arr.ctypes.data_as(_ip), int(arr.size), arr


# ---- generators (rng.rs:20-70, ops/lattice/constants.rs:11-49) -------------
class Lcg:
    """Sequential generator state; arrays are filled in argument order."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def uniform(self, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        lib().bco_fill_uniform(C.byref(self.state), lo, hi, _f(out), out.size)
        return out

    def normal(self, shape, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        lib().bco_fill_normal(C.byref(self.state), mu, sigma, _f(out), out.size)
        return out


def lcg_advance(state: int, inc: int, n: int) -> int:
    return int(lib().bco_lcg_advance(state, inc, n))


# ---- f64 oracles --------------------------------------------------------------
def matmul_f64(a: np.ndarray, b: np.ndarray, rows=None) -> np.ndarray:
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    sp, ns, keep = _sel(rows)
    c = np.empty((ns if rows is not None else m, n), dtype=np.float64)
    lib().bco_matmul_f64(m, n, k, _f(a), k, _f(b), n, _d(c), n, sp, ns)
    return c


def softmax_rows_f64(x: np.ndarray) -> np.ndarray:
    cols = x.shape[-1]
    rows = x.size // cols
    y = np.empty(x.shape, dtype=np.float64)
    lib().bco_softmax_rows_f64(rows, cols, _f(x), _d(y))
    return y


def sdpa_f64(q, k, v, causal: bool, scale: float | None = None, heads=None) -> np.ndarray:
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    sp, ns, keep = _sel(heads)
    o = np.empty((ns, Sq, D) if heads is not None else (B, H, Sq, D), dtype=np.float64)
    lib().bco_sdpa_f64(B, H, Sq, Skv, D, scale, int(causal), _f(q), _f(k), _f(v), _d(o), sp, ns)
    return o


def sdpa_f64_rows(q, k, v, causal: bool, rows, scale: float | None = None) -> np.ndarray:
    """sdpa_f64 on a row sample of every head: rows is [B*H, n] query-row
    indices (per head); returns [B*H, n, D] float64."""
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    r = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
    assert r.ndim == 2 and r.shape[0] == B * H and r.min() >= 0 and r.max() < Sq
    o = np.empty((B * H, r.shape[1], D), dtype=np.float64)
    lib().bco_sdpa_f64_rows(B, H, Sq, Skv, D, scale, int(causal), _f(q), _f(k), _f(v), _d(o),
                            r.ctypes.data_as(_ip), r.shape[1])
    return o


# ---- f32 restatements ---------------------------------------------------------
def matmul_cpu_exec_f32(a, b, row_begin: int = 0, row_end: int | None = None) -> np.ndarray:
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), dtype=np.float32)
    lib().bco_matmul_cpu_exec_f32(m, n, k, _f(a), _f(b), _f(c), row_begin, m if row_end is None else row_end)
    return c


def matmul_k1_f32(a, b) -> np.ndarray:
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=np.float32)
    lib().bco_matmul_k1_f32(m, n, k, _f(a), _f(b), _f(c))
    return c


def batch_matmul_seq_f32(a, b) -> np.ndarray:
    bt, m, k = a.shape
    n = b.shape[2]
    c = np.empty((bt, m, n), dtype=np.float32)
    lib().bco_batch_matmul_seq_f32(bt, m, n, k, _f(a), _f(b), _f(c))
    return c


def softmax_dim_f32(x, axis: int = -1, slice_begin: int = 0, slice_end: int | None = None) -> np.ndarray:
    shape = x.shape
    axis = axis % len(shape)
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    y = np.zeros_like(x)
    end = outer * inner if slice_end is None else slice_end
    lib().bco_softmax_dim_f32(outer, shape[axis], inner, _f(x), _f(y), slice_begin, end)
    return y


def softmax_global_f32(x) -> np.ndarray:
    y = np.empty_like(x)
    lib().bco_softmax_global_f32(x.size, _f(x), _f(y))
    return y


def attention_3pass_f32(q, k, v, causal: bool, heads=None) -> np.ndarray:
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    sp, ns, keep = _sel(heads)
    o = np.empty((ns, Sq, D) if heads is not None else (B, H, Sq, D), dtype=np.float32)
    lib().bco_attention_3pass_f32(B, H, Sq, Skv, D, int(causal), _f(q), _f(k), _f(v), _f(o), sp, ns)
    return o


def causal_attention_cpu_f32(q, k, v, head_begin: int = 0, head_end: int | None = None) -> np.ndarray:
    B, H, S, D = q.shape
    o = np.zeros_like(q)
    lib().bco_causal_attention_cpu_f32(B, H, S, D, _f(q), _f(k), _f(v), _f(o), head_begin,
                                       B * H if head_end is None else head_end)
    return o


# ---- callers of the attention core ------------------------------------------------
def gqa_f64(q, k, v, causal: bool = False, scale: float | None = None) -> np.ndarray:
    """Grouped-query attention in f64 (ops/grouped_query_attention/compute.rs:27-121;
    gqa_matmul_f64.wgsl:44-47 maps query head h to key/value head
    h / heads_per_group, gqa_softmax_f64.wgsl and gqa_apply_f64.wgsl are the
    row softmax and the P.V product of the plain attention).  The K/V heads
    are repeated group-wise (head h of the result reads h // group) and the
    f64 SDPA oracle does the rest.  The reference op is non-causal; causal is
    the same mask as sdpa_f64's."""
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    return sdpa_f64(q, np.repeat(k, g, axis=1), np.repeat(v, g, axis=1), causal, scale)


def gqa_3pass_f32(q, k, v) -> np.ndarray:
    """f32 restatement of the three GQA passes: the same arithmetic as the
    plain attention's K6 -> K7 -> K9 (score = sequential dot / sqrt(D), max
    initialised to -1e9, exp, sum, divide; sequential P.V), with the
    key/value head of query head h being h // (Hq / Hkv)."""
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    return attention_3pass_f32(q, np.ascontiguousarray(np.repeat(k, g, axis=1)),
                               np.ascontiguousarray(np.repeat(v, g, axis=1)), False)


def mha_f64(query, key, value, w_q, w_k, w_v, w_o, num_heads: int) -> np.ndarray:
    """Multi-head attention in float64 throughout (ops/mha/mod.rs:152-187,
    projections.rs:18-58): project with [D, D] weights, split heads
    ([B,S,H*hd] -> [B,H,S,hd] as head_split_f64.wgsl indexes it: element
    (b,h,s,d) <- (b,s,h*hd+d)), non-causal attention with scale 1/sqrt(hd)
    (the Attention op), concatenate heads (head_concat_f64.wgsl, the inverse
    map) and project with W_o."""
    B, Sq, D = query.shape
    Skv = key.shape[1]
    H = num_heads
    hd = D // H
    f = lambda a: np.asarray(a, dtype=np.float64)
    split = lambda x, S: x.reshape(B, S, H, hd).transpose(0, 2, 1, 3)
    qp = split(f(query).reshape(B * Sq, D) @ f(w_q), Sq)
    kp = split(f(key).reshape(B * Skv, D) @ f(w_k), Skv)
    vp = split(f(value).reshape(B * Skv, D) @ f(w_v), Skv)
    s = qp @ kp.transpose(0, 1, 3, 2) / math.sqrt(hd)
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    p = s / s.sum(axis=-1, keepdims=True)
    o = (p @ vp).transpose(0, 2, 1, 3).reshape(B * Sq, D)
    return (o @ f(w_o)).reshape(B, Sq, D)


def linear_f32(x, w_out_in, bias=None, relu: bool = False) -> np.ndarray:
    """linear_f64.wgsl in f32 (see bco_linear_f32): x [batch, in], W [out, in]."""
    batch, in_f = x.shape
    out_f = w_out_in.shape[0]
    y = np.empty((batch, out_f), dtype=np.float32)
    bp = _f(bias) if bias is not None else None
    lib().bco_linear_f32(batch, in_f, out_f, _f(x), _f(w_out_in), bp, int(relu), _f(y))
    return y


def fused_mlp_f32(x, weights, biases) -> np.ndarray:
    """nn/fused_mlp.rs:38-168 in f32 on [out, in] weights: every layer is
    linear_f64.wgsl followed by relu_f64.wgsl, the last one included."""
    for w, b in zip(weights, biases):
        x = linear_f32(np.ascontiguousarray(x), np.ascontiguousarray(w), np.ascontiguousarray(b), True)
    return x


def fused_mlp_f64(x, weights, biases) -> np.ndarray:
    """The fused MLP's mathematical contract in float64: per layer
    y = max(x W^T + b, 0) with W [out, in] (linear_f64.wgsl:33-43 then
    relu_f64.wgsl), ReLU after every layer (fused_mlp.rs:139-151)."""
    y = np.asarray(x, dtype=np.float64)
    for w, b in zip(weights, biases):
        y = np.maximum(y @ np.asarray(w, dtype=np.float64).T + np.asarray(b, dtype=np.float64), 0.0)
    return y


def gemm_f64_wgsl(a, b, m: int, k: int, n: int, batch: int, alpha: float = 1.0, beta: float = 0.0,
                  trans_a: bool = False, trans_b: bool = False, c_in=None) -> np.ndarray:
    """gemm_f64.wgsl restated in C (bco_gemm_f64_wgsl): packed f64 inputs, flat f64 output."""
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float64).reshape(-1)
    c = np.empty(batch * m * n, dtype=np.float64)
    ci = None if c_in is None else _d(np.ascontiguousarray(c_in, dtype=np.float64).reshape(-1))
    lib().bco_gemm_f64_wgsl(int(trans_a), int(trans_b), batch, m, n, k, alpha, _d(a), _d(b), beta, ci, _d(c))
    return c


def gemm_longdouble(a, b, m: int, k: int, n: int, batch: int, trans_a: bool = False,
                    trans_b: bool = False) -> np.ndarray:
    """op(A) op(B) per batch in numpy longdouble (x87 80-bit here): the
    accuracy yardstick for the f64 GEMM, flat output."""
    A = np.asarray(a, dtype=np.longdouble).reshape(batch, k, m) if trans_a else \
        np.asarray(a, dtype=np.longdouble).reshape(batch, m, k)
    B = np.asarray(b, dtype=np.longdouble).reshape(batch, n, k) if trans_b else \
        np.asarray(b, dtype=np.longdouble).reshape(batch, k, n)
    if trans_a:
        A = A.transpose(0, 2, 1)
    if trans_b:
        B = B.transpose(0, 2, 1)
    return np.matmul(A, B).reshape(-1)


# ---- GELU and layer norm (session/mod.rs:349-398) -----------------------------------
def gelu_f64(x) -> np.ndarray:
    """gelu_f64.wgsl:17-31 in float64 (libm tanh)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.float64)
    lib().bco_gelu_f64(x.size, _f(x), _d(y))
    return y


def gelu_wgsl_f32(x) -> np.ndarray:
    """gelu_f64.wgsl downcast to f32 with the tanh builtin (compiler.rs:91-109)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().bco_gelu_wgsl_f32(x.size, _f(x), _f(y))
    return y


def layer_norm_f64(x, eps: float = 1e-5) -> np.ndarray:
    """layer_norm_f64.wgsl:20-50 in float64 over the last axis."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    y = np.empty(x.shape, dtype=np.float64)
    lib().bco_layer_norm_f64(x.size // cols, cols, eps, _f(x), _d(y))
    return y


def layer_norm_f32(x, eps: float = 1e-5) -> np.ndarray:
    """layer_norm_f64.wgsl downcast to f32: sequential sums, one row per thread."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    y = np.empty_like(x)
    lib().bco_layer_norm_f32(x.size // cols, cols, eps, _f(x), _f(y))
    return y


# ---- inline-data f64 handlers (barracuda-core/src/ipc/methods/) --------------------
def ml_softmax_rows_f64(x) -> np.ndarray:
    """ml/forward.rs:130-140 on each row of a float64 matrix: f64::max fold
    from -inf, exp(x - max), sequential sum, divide."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    cols = x.shape[-1]
    y = np.empty_like(x)
    lib().bco_ml_softmax_rows_f64(x.size // cols, cols, _d(x), _d(y))
    return y


def ml_attention_f64(q, k, v) -> np.ndarray:
    """ml/forward.rs:121-150: softmax(Q K^T / sqrt(d_k)) V in float64, the
    handler's own operation order."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float64) for a in (q, k, v))
    (sq, dk), (sk, dv) = q.shape, v.shape
    assert k.shape == (sk, dk)
    out = np.empty((sq, dv), dtype=np.float64)
    lib().bco_ml_attention_f64(sq, sk, dk, dv, _d(q), _d(k), _d(v), _d(out))
    return out


def matmul_inline_f64(lhs, rhs) -> np.ndarray:
    """tensor.rs:540-548: sum = lhs[i][p].mul_add(rhs[p][j], sum) over p."""
    lhs, rhs = (np.ascontiguousarray(a, dtype=np.float64) for a in (lhs, rhs))
    (m, k), (k2, n) = lhs.shape, rhs.shape
    assert k == k2
    out = np.empty((m, n), dtype=np.float64)
    lib().bco_matmul_inline_f64(m, k, n, _d(lhs), _d(rhs), _d(out))
    return out


# ---- metric (tolerances/mod.rs:44-54 scale) ---------------------------------------
def max_rel_err(x: np.ndarray, ref: np.ndarray) -> float:
    """max |x - ref| / max(|ref|, 1); non-finite values must match exactly."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if ref.dtype == np.float64:
        ref = np.ascontiguousarray(ref).reshape(-1)
        return float(lib().bco_max_rel_err(x.size, _f(x), _d(ref)))
    ref = np.ascontiguousarray(ref, dtype=np.float32).reshape(-1)
    return float(lib().bco_max_rel_err_f32ref(x.size, _f(x), _f(ref)))


def num_threads() -> int:
    return int(lib().bco_num_threads())


def set_num_threads(n: int) -> None:
    """Threads of the OpenMP loops from now on (n >= 1)."""
    lib().bco_set_num_threads(int(n))
