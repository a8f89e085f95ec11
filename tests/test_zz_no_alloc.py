"""bch_sgemm_noalloc (the matmul entry point that allocates nothing; its
scratch is a fixed per-GPU device array) against bch_sgemm, called through
the C ABI: bit-identical outputs, on two calls in a row with the second
smaller, on each kernel family (decode-shaped split-k paths that use the
scratch, the MFMA tile path that needs none, the tile path's split-K and
hybrid plan over the scratch); the whole tiles where the hybrid plan's
partials exceed the scratch; and a clear rejection of a shape whose
required partials would not fit.  The property itself -- no allocation --
is tested on fresh contexts (workspace never grown) whose first call is
the no-alloc one, made under a global-mode stream capture (where an
allocation fails), replayed and compared with bch_sgemm; the fresh
context's workspace must still be empty afterwards."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import Tensor
from barracuda_amd import _native as N
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _both(dev, m, n, k, seed):
    rng = O.Lcg(seed)
    a, b = rng.normal((m, k)), rng.normal((k, n), 0.0, 0.02)
    ta, tb = Tensor.from_data(a, [m, k], dev), Tensor.from_data(b, [k, n], dev)
    c_ref, c_na = Tensor.empty([m, n], dev), Tensor.empty([m, n], dev)
    lib, ctx = dev._lib, dev.ctx
    pa, pb = C.c_void_p(ta.ptr), C.c_void_p(tb.ptr)
    dev.check(lib.bch_sgemm(ctx, m, n, k, pa, k, pb, n, C.c_void_p(c_ref.ptr), n), "sgemm")
    dev.check(lib.bch_sgemm_noalloc(ctx, m, n, k, pa, k, pb, n, C.c_void_p(c_na.ptr), n), "sgemm_noalloc")
    got, want = c_na.to_numpy(), c_ref.to_numpy()
    return got, want, a, b


@pytest.mark.parametrize("shapes", [
    # (m, n, k) pairs: a call, then a smaller one; decode paths use the scratch
    [(32, 11008, 4096), (8, 3000, 1024)],
    [(8, 11008, 4096), (1, 4096, 512)],
    [(1, 11008, 4096), (20, 1000, 300)],
    [(256, 512, 384), (32, 256, 64)],
    # split-K (slices in the scratch, then the reduce), then a smaller split
    [(1024, 1024, 4096), (96, 1024, 2048)],
    # the hybrid plan (16 MiB and 8.5 MiB of tail partials in the scratch)
    [(3072, 3072, 1024), (2304, 2304, 1024)],
])
def test_noalloc_matches_sgemm_twice(dev, shapes):
    for i, (m, n, k) in enumerate(shapes):
        _say(f"sgemm_noalloc call {i}: m={m} n={n} k={k} kernel={dev._lib.bch_sgemm_kernel_name(m, n, k).decode()}")
        got, want, a, b = _both(dev, m, n, k, 1000 * i + m + n + k)
        assert np.array_equal(got, want), (m, n, k)
        rows = list(range(min(m, 4))) + [m - 1]
        assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL


def test_noalloc_takes_whole_tiles_where_the_hybrid_does_not_fit(dev):
    """6144 x 6144 x 1536 takes the hybrid plan through bch_sgemm (64 MiB of tail partials,
    more than the fixed scratch); the no-alloc call runs whole tiles instead, then a smaller
    hybrid shape that fits.  Each within tolerance of bch_sgemm and of f64."""
    for i, (m, n, k) in enumerate(((6144, 6144, 1536), (3000, 3000, 1024))):
        _say(f"sgemm_noalloc call {i}: m={m} n={n} k={k} (bch_sgemm: {dev._lib.bch_sgemm_kernel_name(m, n, k).decode()})")
        got, want, a, b = _both(dev, m, n, k, 7000 + i)
        assert O.max_rel_err(got, want.astype(np.float64)) <= TOL
        rows = [0, 1, m // 2, m - 1]
        assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL


def test_noalloc_takes_fewer_slices_where_the_split_does_not_fit(dev):
    """128 x 11008 x 4096 splits K 8 ways through bch_sgemm (45 MB of partials, more than the
    fixed scratch); the no-alloc call plans within the scratch (2 slices), then a smaller split
    shape.  Each within tolerance of bch_sgemm and of f64."""
    for i, (m, n, k) in enumerate(((128, 11008, 4096), (96, 4096, 4096))):
        _say(f"sgemm_noalloc call {i}: m={m} n={n} k={k} (bch_sgemm: {dev._lib.bch_sgemm_kernel_name(m, n, k).decode()})")
        got, want, a, b = _both(dev, m, n, k, 8000 + i)
        assert O.max_rel_err(got, want.astype(np.float64)) <= TOL
        rows = [0, 1, m // 2, m - 1]
        assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL


def test_noalloc_takes_the_tiles_where_64_row_skinny_partials_do_not_fit(dev):
    """64 x 11008 x 4096 runs the 64-row skinny kernel through bch_sgemm (about 20 MB of split-k
    partials, more than the fixed scratch); the no-alloc call takes the tile path, then a smaller
    64-row skinny shape whose partials fit.  Each within tolerance of bch_sgemm and of f64."""
    for i, (m, n, k) in enumerate(((64, 11008, 4096), (48, 4096, 1024))):
        _say(f"sgemm_noalloc call {i}: m={m} n={n} k={k} (bch_sgemm: {dev._lib.bch_sgemm_kernel_name(m, n, k).decode()})")
        got, want, a, b = _both(dev, m, n, k, 9000 + i)
        assert O.max_rel_err(got, want.astype(np.float64)) <= TOL
        rows = [0, 1, m // 2, m - 1]
        assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL


def test_noalloc_rejects_what_does_not_fit(dev):
    """m = 32, n = 262144: the split-k partials exceed the fixed 16 MiB, so
    the call fails before any launch, with the sizes in the message."""
    m, n, k = 32, 262144, 64
    _say(f"sgemm_noalloc rejection m={m} n={n} k={k}")
    ta, tb, tc = Tensor.empty([m, k], dev), Tensor.empty([k, n], dev), Tensor.empty([m, n], dev)
    lib = dev._lib
    st = lib.bch_sgemm_noalloc(dev.ctx, m, n, k, C.c_void_p(ta.ptr), k, C.c_void_p(tb.ptr), n,
                               C.c_void_p(tc.ptr), n)
    assert st == N.BCH_E_UNSUPPORTED
    msg = N.last_error(dev.ctx)
    assert "scratch" in msg and str(16 << 20) in msg
    # the context stays usable
    dev.sync()


HIP_LIB = "/opt/rocm/lib/libamdhip64.so.7"  # the runtime libbarracuda_hip.so is linked against
CAPTURE_GLOBAL = 0                           # hipStreamCaptureModeGlobal


def _hip():
    h = C.CDLL(HIP_LIB)
    h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    h.hipGraphExecDestroy.argtypes = [C.c_void_p]
    h.hipGraphDestroy.argtypes = [C.c_void_p]
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(h, f).restype = C.c_int
    return h


@pytest.mark.parametrize("family,shapes", [
    ("skinny split-k m=32 then m=8", [(32, 11008, 4096), (8, 3000, 1024)]),
    ("skinny fma m=1 then m=20", [(1, 11008, 4096), (20, 1000, 300)]),
    ("tiles (no scratch) then skinny", [(256, 512, 384), (32, 256, 64)]),
    ("split-K then a smaller split", [(1024, 1024, 4096), (96, 1024, 2048)]),
    ("hybrid plan then a smaller hybrid", [(3072, 3072, 1024), (2304, 2304, 1024)]),
])
def test_noalloc_allocates_nothing_under_global_capture(dev, family, shapes):
    hip = _hip()
    lib = dev._lib
    for i, (m, n, k) in enumerate(shapes):
        _say(f"sgemm_noalloc captured on a fresh context ({family}), call {i}: m={m} n={n} k={k}")
        rng = O.Lcg(500 + 1000 * i + m + n + k)
        a, b = rng.normal((m, k)), rng.normal((k, n), 0.0, 0.02)
        ta, tb = Tensor.from_data(a, [m, k], dev), Tensor.from_data(b, [k, n], dev)
        c_ref, c_na = Tensor.empty([m, n], dev), Tensor.empty([m, n], dev)
        pa, pb = C.c_void_p(ta.ptr), C.c_void_p(tb.ptr)
        dev.check(lib.bch_sgemm(dev.ctx, m, n, k, pa, k, pb, n, C.c_void_p(c_ref.ptr), n), "sgemm")
        want = c_ref.to_numpy()
        ctx, stream = C.c_void_p(), C.c_void_p()
        assert lib.bch_ctx_create(0, None, C.byref(ctx)) == N.BCH_OK
        graph, exe = C.c_void_p(), C.c_void_p()
        try:
            assert lib.bch_ctx_stream(ctx, C.byref(stream)) == N.BCH_OK
            ws = C.c_size_t(1)
            assert lib.bch_ctx_workspace_bytes(ctx, C.byref(ws)) == N.BCH_OK and ws.value == 0
            assert hip.hipStreamBeginCapture(stream, CAPTURE_GLOBAL) == 0
            st = lib.bch_sgemm_noalloc(ctx, m, n, k, pa, k, pb, n, C.c_void_p(c_na.ptr), n)
            assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
            assert st == N.BCH_OK, N.last_error(ctx)
            assert lib.bch_ctx_workspace_bytes(ctx, C.byref(ws)) == N.BCH_OK and ws.value == 0
            assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
            for rep in range(2):
                dev.upload(c_na.ptr, np.full((m, n), np.nan, np.float32))
                assert hip.hipGraphLaunch(exe, stream) == 0
                assert lib.bch_sync(ctx) == N.BCH_OK
                got = c_na.to_numpy()
                assert np.array_equal(got, want), (family, rep)  # the same kernels and plan as bch_sgemm
                rows = list(range(min(m, 4))) + [m - 1]
                assert O.max_rel_err(got[rows], O.matmul_f64(a, b, rows=rows)) <= TOL
            assert lib.bch_ctx_workspace_bytes(ctx, C.byref(ws)) == N.BCH_OK and ws.value == 0
        finally:
            if exe.value:
                hip.hipGraphExecDestroy(exe)
            if graph.value:
                hip.hipGraphDestroy(graph)
            lib.bch_ctx_destroy(ctx)
