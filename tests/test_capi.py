"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and validates arguments/shapes before touching a device
(include/barracuda_hip.h conventions).  Also the host-side op API's shape
validation, which mirrors the reference's error variants."""
from __future__ import annotations

import ctypes as C
import subprocess

import numpy as np
import pytest

from barracuda_amd import _native as N
from barracuda_amd.error import (DeviceNotAvailable, InvalidOperation, OutOfMemory, ShapeMismatch,
                                 UnsupportedOperation, from_status)


def test_library_exports_every_header_symbol():
    syms = N.header_symbols()
    assert len(syms) >= 20
    lib = N.load()
    for s in syms:
        assert hasattr(lib, s), s
    # the binding declares a signature for each exported function
    assert set(syms) == set(N.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(syms) <= exported


def test_rust_binding_in_integration_doc_matches_header():
    """The barracuda-hip-sys block a maintainer would paste (the integration guide at the
    repository root) declares exactly the header's functions and status codes."""
    import re
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    doc = (root / "INTEGRATION.md").read_text()
    block = re.search(r'extern "C" \{(.*?)\n\}', doc, re.S).group(1)
    assert set(re.findall(r"pub fn (bch_[a-z0-9_]+)", block)) == set(N.header_symbols())
    header = (root / "include" / "barracuda_hip.h").read_text()
    codes = dict(re.findall(r"#define (BCH_(?:OK|E_[A-Z_]+))\s+(\d+)", header))
    rust = dict(re.findall(r"pub const (BCH_(?:OK|E_[A-Z_]+)): bch_status = (\d+);", doc))
    assert codes and rust == codes
    for code in codes:  # every status has a row in the error-mapping table (BCH_OK excepted)
        assert code == "BCH_OK" or f"| `{code}` |" in doc, code


def test_library_carries_gfx950_code():
    # the fat binary embedded in our own build names its target
    assert b"amdgcn-amd-amdhsa--gfx950" in N.LIB_PATH.read_bytes()
    hsaco = N.PKG / "lib" / "bch_softmax_rows.hsaco"
    assert hsaco.exists() and hsaco.read_bytes()[:4] == b"\x7fELF"


def test_status_strings_and_no_device_behaviour():
    lib = N.load()
    assert lib.bch_status_string(N.BCH_OK) == b"ok"
    assert lib.bch_status_string(N.BCH_E_SHAPE) == b"shape mismatch"
    assert lib.bch_status_string(99) == b"unknown status"
    n = C.c_int(-1)
    st = lib.bch_device_count(C.byref(n))
    if st == N.BCH_E_NO_DEVICE:  # this container: no GPU
        assert n.value == 0
        ctx = C.c_void_p()
        assert lib.bch_ctx_create(0, None, C.byref(ctx)) == N.BCH_E_NO_DEVICE
        assert ctx.value is None
        assert "no HIP device" in N.last_error(None)
        with pytest.raises(DeviceNotAvailable):
            from barracuda_amd import HipDevice
            HipDevice(0)
    else:
        assert st == N.BCH_OK and n.value >= 1


def test_null_and_shape_errors_before_device():
    lib = N.load()
    nul = C.c_void_p()
    assert lib.bch_device_count(None) == N.BCH_E_INVALID
    assert lib.bch_ctx_create(0, None, None) == N.BCH_E_INVALID
    # shapes are validated first, identically with or without a GPU
    assert lib.bch_sgemm(nul, -1, 4, 4, nul, 4, nul, 4, nul, 4) == N.BCH_E_SHAPE
    assert "negative dimension" in N.last_error(None)
    assert lib.bch_sgemm(nul, 4, 4, 8, nul, 4, nul, 4, nul, 4) == N.BCH_E_SHAPE  # lda < k
    assert "leading dimension" in N.last_error(None)
    assert lib.bch_sgemm(nul, 4, 4, 4, nul, 4, nul, 4, nul, 4) == N.BCH_E_INVALID  # ctx NULL
    assert lib.bch_sgemm_strided_batched(nul, 2, 4, 4, 4, nul, 8, nul, 16, nul, 16) == N.BCH_E_SHAPE
    assert lib.bch_softmax_rows(nul, 0, 5, nul, nul) == N.BCH_E_SHAPE
    assert lib.bch_softmax_rows(nul, 2, 5, nul, nul) == N.BCH_E_INVALID
    assert lib.bch_softmax_axis(nul, 1, 0, 1, nul, nul) == N.BCH_E_SHAPE
    assert lib.bch_sdpa_fwd(nul, 1, 1, 4, 8, 16, 0.25, 1, nul, nul, nul, nul) == N.BCH_E_SHAPE
    assert "causal" in N.last_error(None)
    # any head dimension is accepted (the reference's ops take any); only the NULL ctx fails here
    assert lib.bch_sdpa_fwd(nul, 1, 1, 4, 4, 512, 0.25, 0, nul, nul, nul, nul) == N.BCH_E_INVALID
    assert "ctx is NULL" in N.last_error(None)
    assert lib.bch_sdpa_fwd(nul, 0, 1, 4, 4, 16, 0.25, 0, nul, nul, nul, nul) == N.BCH_E_SHAPE
    grid = (C.c_uint * 3)(1, 1, 1)
    assert lib.bch_launch_code_object(nul, None, 0, b"x", grid, grid, None, 0, 0) == N.BCH_E_INVALID
    ev = C.c_void_p()
    assert lib.bch_event_create(nul, C.byref(ev)) == N.BCH_E_INVALID
    f = C.c_float()
    assert lib.bch_event_elapsed_ms(nul, nul, C.byref(f)) == N.BCH_E_INVALID
    lib.bch_ctx_destroy(nul)  # NULL is a no-op
    lib.bch_event_destroy(nul)


def test_kernel_routing_names():
    lib = N.load()
    assert lib.bch_sgemm_kernel_name(4096, 4096, 4096) == b"sgemm_mfma_kernel<256,256,32,false>"
    assert lib.bch_sgemm_kernel_name(3072, 3072, 512) == b"sgemm_mfma_kernel<128,128,32,false,hyb>+sgemm_tail_reduce"
    assert lib.bch_sgemm_kernel_name(2048, 2048, 512) == b"sgemm_mfma_kernel<128,128,32,false>"
    assert lib.bch_sgemm_kernel_name(3000, 3000, 1000) == b"sgemm_mfma_kernel<128,128,32,true,v4>"
    assert lib.bch_sgemm_kernel_name(8192, 1024, 512) == b"sgemm_mfma_kernel<256,128,32,false>"
    assert lib.bch_sgemm_kernel_name(4096, 11008, 4096) == (b"sgemm_mfma_kernel<256,256,32,false> columns then "
                                                            b"sgemm_mfma_kernel<128,128,32,false>")
    assert lib.bch_sgemm_kernel_name(11008, 4096, 4096) == (b"sgemm_mfma_kernel<256,256,32,false> rows then "
                                                            b"sgemm_mfma_kernel<128,128,32,false>")
    assert lib.bch_sgemm_kernel_name(3072, 3072, 3072) == b"sgemm_mfma_kernel<256,128,32,false,hyb>+sgemm_tail_reduce"
    assert lib.bch_sgemm_kernel_name(1024, 1024, 1024) == b"sgemm_mfma_kernel<64,64,64,false>"
    assert lib.bch_sgemm_kernel_name(1024, 1024, 4096) == b"sgemm_mfma_kernel<128,128,32,false>+sgemm_splitk_reduce"
    assert lib.bch_sgemm_kernel_name(2048, 2048, 2048) == b"sgemm_mfma_kernel<128,128,32,false>"
    assert lib.bch_sgemm_kernel_name(4100, 4096, 300) == b"sgemm_mfma_kernel<128,128,32,true,v4>"
    assert lib.bch_sgemm_kernel_name(4000, 4000, 4000) == b"sgemm_mfma_kernel<256,256,32,true,v4>"
    assert lib.bch_sgemm_kernel_name(1, 11008, 4096) == b"sgemm_skinny_fma"
    assert lib.bch_sgemm_kernel_name(8, 11008, 4096) == b"sgemm_skinny_sk<1>"
    assert lib.bch_sgemm_kernel_name(16, 11008, 4096) == b"sgemm_skinny_sk<1>"
    assert lib.bch_sgemm_kernel_name(32, 11008, 4096) == b"sgemm_skinny_w32"
    assert lib.bch_sgemm_kernel_name(100, 70, 33) == b"sgemm_mfma_kernel<128,128,32,true>"


def test_status_to_error_variant_mapping():
    assert isinstance(from_status(N.BCH_E_SHAPE, "x", "matmul"), InvalidOperation)
    assert "mismatch" in str(from_status(N.BCH_E_SHAPE, "x", "matmul"))
    assert isinstance(from_status(N.BCH_E_OOM, "x"), OutOfMemory)
    assert isinstance(from_status(N.BCH_E_NO_DEVICE, "x"), DeviceNotAvailable)
    assert str(from_status(N.BCH_E_NO_DEVICE, "no GPU", device="hip")) == "Device not available: hip - no GPU"
    assert isinstance(from_status(N.BCH_E_UNSUPPORTED, "x"), UnsupportedOperation)
    from barracuda_amd.error import DeviceError, DeviceLost, ExecutionError, InvalidInput
    assert isinstance(from_status(N.BCH_E_LAUNCH, "x"), ExecutionError)
    assert isinstance(from_status(N.BCH_E_INVALID, "x"), InvalidInput)
    for st in (N.BCH_E_MODULE, N.BCH_E_DEVICE):
        e = from_status(st, "x")
        assert isinstance(e, DeviceError) and not isinstance(e, DeviceLost)
    lost = from_status(N.BCH_E_DEVICE_LOST, "fault")
    assert isinstance(lost, DeviceLost) and str(lost) == "GPU device lost: fault"  # error.rs:59


def test_device_lost_status_string_and_null_query():
    import ctypes as C
    lib = N.load()
    assert lib.bch_status_string(N.BCH_E_DEVICE_LOST) == b"device lost"
    flag = C.c_int(5)
    assert lib.bch_ctx_is_lost(None, C.byref(flag)) == N.BCH_E_INVALID


class _FakeTensor:
    """Shape-only stand-in: the op constructors validate before any device work."""

    def __init__(self, shape):
        self._shape = list(shape)

    def shape(self):
        return list(self._shape)

    def device(self):
        return None


def test_op_api_shape_validation_mirrors_reference():
    from barracuda_amd import (Attention, CausalAttention, FlashAttention, InvalidInput, MatMul,
                               ScaledDotProductAttention, Softmax)
    T = _FakeTensor
    # matmul.rs:92-114
    with pytest.raises(InvalidOperation, match="2D"):
        MatMul(T([4]), T([4, 4])).execute()
    with pytest.raises(ShapeMismatch) as e:
        MatMul(T([2, 3]), T([4, 2])).execute()
    assert "mismatch" in str(e.value).lower()  # fault_injection.rs:46-55 wording
    # softmax.rs:39-48
    with pytest.raises(InvalidOperation, match="Empty tensor"):
        Softmax(T([]))
    # attention/mod.rs:96-144
    with pytest.raises(InvalidOperation, match="4D"):
        Attention(T([2, 4, 8]), T([1, 2, 4, 8]), T([1, 2, 4, 8]))
    with pytest.raises(ShapeMismatch):
        Attention(T([1, 2, 4, 8]), T([1, 3, 4, 8]), T([1, 3, 4, 8]))
    with pytest.raises(ShapeMismatch):
        Attention(T([1, 2, 4, 8]), T([1, 2, 6, 8]), T([1, 2, 5, 8]))
    Attention(T([1, 2, 4, 8]), T([1, 2, 6, 8]), T([1, 2, 6, 8]))  # cross-attention is fine
    # sdpa/mod.rs:101-149
    with pytest.raises(InvalidInput):
        ScaledDotProductAttention(T([4, 8]), T([4, 8]), T([4, 8]))
    with pytest.raises(ShapeMismatch):
        ScaledDotProductAttention(T([1, 1, 4, 8]), T([1, 1, 5, 8]), T([1, 1, 4, 8]))
    # causal_attn/mod.rs:78-95
    with pytest.raises(ShapeMismatch):
        CausalAttention(T([1, 1, 4, 8]), T([1, 1, 4, 8]), T([1, 1, 4, 4]))
    # flash_attention.rs:57-80
    with pytest.raises(InvalidOperation, match="same shape"):
        FlashAttention(T([4, 8]), T([4, 4]), T([4, 8]), 1)
    with pytest.raises(InvalidOperation, match="2D"):
        FlashAttention(T([1, 4, 8]), T([1, 4, 8]), T([1, 4, 8]), 1)


def test_sdpa_ex_validation_before_device():
    lib = N.load()
    nul = C.c_void_p()
    dense = N.AttnLayout(8 * 16 * 32, 16 * 32, 32)
    # num_q_heads must be a multiple of num_kv_heads (grouped_query_attention/mod.rs:118-123)
    assert lib.bch_sdpa_fwd_ex(nul, 1, 8, 3, 16, 16, 32, 0.25, 0, nul, dense, nul, dense, nul, dense, nul,
                               dense) == N.BCH_E_INVALID
    assert "num_q_heads (8) must be divisible by num_kv_heads (3)" in N.last_error(None)
    assert lib.bch_sdpa_fwd_ex(nul, 1, 8, 0, 16, 16, 32, 0.25, 0, nul, dense, nul, dense, nul, dense, nul,
                               dense) == N.BCH_E_SHAPE
    bad = N.AttnLayout(0, 0, 16)  # row stride < D
    assert lib.bch_sdpa_fwd_ex(nul, 1, 8, 2, 16, 16, 32, 0.25, 0, nul, dense, nul, bad, nul, dense, nul,
                               dense) == N.BCH_E_INVALID
    assert "k layout" in N.last_error(None)
    assert lib.bch_sdpa_fwd_ex(nul, 1, 8, 2, 16, 8, 32, 0.25, 1, nul, dense, nul, dense, nul, dense, nul,
                               dense) == N.BCH_E_SHAPE
    assert lib.bch_sdpa_fwd_ex(nul, 1, 8, 2, 16, 16, 32, 0.25, 0, nul, dense, nul, dense, nul, dense, nul,
                               dense) == N.BCH_E_INVALID  # ctx NULL


def test_sgemm_ex_validation_before_device():
    lib = N.load()
    nul = C.c_void_p()
    assert lib.bch_sgemm_ex(nul, 2, 4, 4, 4, nul, 4, nul, 4, nul, 0, nul, 4) == N.BCH_E_INVALID
    assert "transb" in N.last_error(None)
    assert lib.bch_sgemm_ex(nul, 0, 4, 4, 4, nul, 4, nul, 4, nul, 7, nul, 4) == N.BCH_E_INVALID
    assert "activation" in N.last_error(None)
    # transb: B is [n, k], so ldb >= k
    assert lib.bch_sgemm_ex(nul, 1, 4, 16, 8, nul, 8, nul, 4, nul, N.BCH_ACT_RELU, nul, 16) == N.BCH_E_SHAPE
    assert "leading dimension" in N.last_error(None)
    assert lib.bch_sgemm_ex(nul, 0, 4, 16, 8, nul, 8, nul, 8, nul, N.BCH_ACT_RELU, nul, 16) == N.BCH_E_SHAPE
    assert lib.bch_sgemm_ex(nul, 1, 4, 16, 8, nul, 8, nul, 8, nul, N.BCH_ACT_RELU, nul, 16) == N.BCH_E_INVALID


def test_dgemm_validation_before_device():
    lib = N.load()
    nul = C.c_void_p()
    assert lib.bch_dgemm(nul, 2, 0, 1, 4, 4, 4, 1.0, nul, 4, 16, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_INVALID
    assert lib.bch_dgemm(nul, 0, 0, 1, -1, 4, 4, 1.0, nul, 4, 16, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_SHAPE
    # transa: A stored [k][m], lda >= m
    assert lib.bch_dgemm(nul, 1, 0, 1, 8, 4, 2, 1.0, nul, 2, 16, nul, 4, 8, 0.0, nul, 4, 32) == N.BCH_E_SHAPE
    assert "leading dimension" in N.last_error(None)
    assert lib.bch_dgemm(nul, 0, 0, 2, 4, 4, 4, 1.0, nul, 4, 8, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_SHAPE
    assert "batch stride" in N.last_error(None)
    assert lib.bch_dgemm(nul, 1, 1, 2, 4, 4, 4, 1.0, nul, 4, 16, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_INVALID


def test_dgemm_empty_k_batched_passes_validation():
    """Batched GemmF64 with k == 0 (packed strides m*k = 0, k*n = 0, lda =
    ldb-of-B^T = 1): A and B are empty, so only C's stride is checked and
    validation reaches the ctx check (BCH_E_INVALID with ctx = NULL), as the
    reference only rejects length mismatches (ops/linalg/gemm_f64.rs)."""
    lib = N.load()
    nul = C.c_void_p()
    # transa = transb = 0: lda = max(k, 1), strideA = m*k = 0, strideB = k*n = 0
    assert lib.bch_dgemm(nul, 0, 0, 3, 4, 5, 0, 1.0, nul, 1, 0, nul, 5, 0, 0.5, nul, 5, 20) == N.BCH_E_INVALID
    assert "ctx" in N.last_error(None)
    # trans_b with k == 0: B stored [n][k], ldb = 1
    assert lib.bch_dgemm(nul, 0, 1, 3, 4, 5, 0, 1.0, nul, 1, 0, nul, 1, 0, 0.5, nul, 5, 20) == N.BCH_E_INVALID
    # transa with k == 0: A stored [k][m] is empty
    assert lib.bch_dgemm(nul, 1, 0, 3, 4, 5, 0, 1.0, nul, 4, 0, nul, 5, 0, 0.5, nul, 5, 20) == N.BCH_E_INVALID
    # C's stride is still checked
    assert lib.bch_dgemm(nul, 0, 0, 3, 4, 5, 0, 1.0, nul, 1, 0, nul, 5, 0, 0.5, nul, 5, 19) == N.BCH_E_SHAPE
    # padded leading dimensions: the extent is (rows - 1) * ld + row length
    assert lib.bch_dgemm(nul, 0, 0, 2, 4, 4, 4, 1.0, nul, 6, 22, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_INVALID
    assert lib.bch_dgemm(nul, 0, 0, 2, 4, 4, 4, 1.0, nul, 6, 21, nul, 4, 16, 0.0, nul, 4, 16) == N.BCH_E_SHAPE


def test_sgemm_noalloc_validation_before_device():
    """The no-allocation matmul validates like bch_sgemm before the context
    is needed."""
    lib = N.load()
    nul = C.c_void_p()
    assert lib.bch_sgemm_noalloc(nul, -1, 4, 4, nul, 4, nul, 4, nul, 4) == N.BCH_E_SHAPE
    assert lib.bch_sgemm_noalloc(nul, 4, 4, 4, nul, 3, nul, 4, nul, 4) == N.BCH_E_SHAPE
    assert "leading dimension" in N.last_error(None)
    assert lib.bch_sgemm_noalloc(nul, 4, 4, 4, nul, 4, nul, 4, nul, 4) == N.BCH_E_INVALID
    assert "ctx" in N.last_error(None)


def test_softmax_f64_validation_and_routing_before_device():
    lib = N.load()
    nul = None
    assert lib.bch_softmax_rows_f64(nul, 0, 4, nul, nul) == N.BCH_E_SHAPE
    assert lib.bch_softmax_rows_f64(nul, 4, 0, nul, nul) == N.BCH_E_SHAPE
    assert lib.bch_softmax_rows_f64(nul, 1 << 31, 4, nul, nul) == N.BCH_E_INVALID  # any row count; ctx NULL
    assert lib.bch_softmax_rows_f64(nul, 4, 4, nul, nul) == N.BCH_E_INVALID
    name = lambda r, c, p: lib.bch_softmax_rows_f64_kernel_name(r, c, C.c_void_p(p), C.c_void_p(p))
    assert name(65536, 2048, 0x1000) == b"softmax_f64_rows<4,2,4>"
    assert name(65536, 2048, 0x1008) == b"softmax_f64_rows<8,1,4>"
    assert name(3, 5, 0x1000) == b"softmax_f64_rows<1,1,1>"
    assert name(3, 129, 0x1000) == b"softmax_f64_rows<4,1,1>"
    assert name(3, 2049, 0x1000) == b"softmax_f64_rows<16,1,4>"
    assert name(3, 8192, 0x1000) == b"softmax_f64_rows<16,2,4>"
    assert name(3, 8193, 0x1000) == b"softmax_f64_block"


def test_elementwise_and_layer_norm_validation_before_device():
    lib = N.load()
    nul = C.c_void_p()
    assert lib.bch_elementwise(nul, 8, 4, nul, nul, nul, 0.0, nul) == N.BCH_E_INVALID
    assert "unknown op" in N.last_error(None)
    assert lib.bch_elementwise(nul, N.BCH_EW_ADD, -1, nul, nul, nul, 0.0, nul) == N.BCH_E_SHAPE
    assert lib.bch_elementwise(nul, N.BCH_EW_GELU, 4, nul, nul, nul, 0.0, nul) == N.BCH_E_INVALID
    assert lib.bch_layer_norm(nul, 0, 4, 1e-5, nul, nul) == N.BCH_E_SHAPE
    assert lib.bch_layer_norm(nul, 4, 4, -1.0, nul, nul) == N.BCH_E_INVALID
    assert lib.bch_layer_norm(nul, 4, 4, float("nan"), nul, nul) == N.BCH_E_INVALID
    assert lib.bch_layer_norm(nul, 1 << 31, 4, 1e-5, nul, nul) == N.BCH_E_INVALID  # any row count; ctx NULL
    assert lib.bch_layer_norm(nul, 4, 4, 1e-5, nul, nul) == N.BCH_E_INVALID
    assert "ctx" in N.last_error(None)
    assert lib.bch_sgemm_ex(nul, 0, 4, 4, 4, nul, 4, nul, 4, nul, 3, nul, 4) == N.BCH_E_INVALID
    assert lib.bch_sgemm_ex(nul, 1, 4, 4, 4, nul, 4, nul, 4, nul, N.BCH_ACT_GELU, nul, 4) == N.BCH_E_INVALID
    assert "ctx" in N.last_error(None)
    # the name follows the buffers' alignment, as the launch does
    name = lambda r, c, p=0x1000, q=None: lib.bch_layer_norm_kernel_name(r, c, C.c_void_p(p),
                                                                         C.c_void_p(p if q is None else q))
    assert name(65536, 2048) == b"layer_norm_wave<8>"
    assert name(3, 4100) == b"layer_norm_wg<8>"
    assert name(3, 32768) == b"layer_norm_wg<32>"
    assert name(3, 32772) == b"layer_norm_wg<16, 1024>"
    assert name(3, 65540) == b"layer_norm_block"
    assert name(3, 4099) == b"layer_norm_wgs<16, 1024>"
    assert name(3, 32771) == b"layer_norm_block"
    # one float off 16-byte alignment (input or output): the scalar register kernels
    assert name(65536, 2048, 0x1004) == b"layer_norm_wgs<16, 256>"
    assert name(65536, 2048, 0x1000, 0x2004) == b"layer_norm_wgs<16, 256>"
    assert name(3, 8192, 0x1004) == b"layer_norm_wgs<16, 1024>"
    assert name(3, 32768, 0x1004) == b"layer_norm_wgs<32, 1024>"
    assert name(3, 65536, 0x1004) == b"layer_norm_block"
