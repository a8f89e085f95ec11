"""HIP graph capture of the library's calls on a context's stream (bch_ctx_stream).

Captured: the decode linear layer with [out, in] weights (the ring kernel, whose
split-k blocks are combined in the kernel through epoch flags that every launch
resets; at m = 48 in two passes), the skinny GEMM (main kernel + reduce; the one-
and two-block kernels), the tile GEMM's hybrid plan (whole tiles and k-slices in
one launch + reduce) and its split-K (slices into the workspace + reduce), row
softmax and attention.  The graph is replayed several times with the program's
own eager calls (which reuse the same workspace and flags) and synchronisations
between the replays; every replay must reproduce the eager results bit for bit.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from barracuda_amd import Tensor
from barracuda_amd import _native as N
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu

HIP_LIB = "/opt/rocm/lib/libamdhip64.so.7"  # the runtime libbarracuda_hip.so is linked against
CAPTURE_RELAXED = 2                          # hipStreamCaptureModeRelaxed
CAPTURE_GLOBAL = 0                           # hipStreamCaptureModeGlobal


def _say(msg):
    print(msg, flush=True)


def _hip():
    h = C.CDLL(HIP_LIB)
    h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    h.hipGraphExecDestroy.argtypes = [C.c_void_p]
    h.hipGraphDestroy.argtypes = [C.c_void_p]
    h.hipGraphGetNodes.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_size_t)]
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphExecDestroy", "hipGraphDestroy", "hipGraphGetNodes"):
        getattr(h, f).restype = C.c_int
    return h


def _up(dev, a):
    return Tensor.from_data(np.ascontiguousarray(a, dtype=np.float32), list(a.shape), dev)


def test_graph_replays_match_eager(dev):
    _say("graph capture: decode linear, skinny GEMM, softmax, attention")
    hip = _hip()
    lib = dev._lib
    stream = C.c_void_p()
    dev.check(lib.bch_ctx_stream(dev.ctx, C.byref(stream)), "ctx_stream")
    assert stream.value

    rng = O.Lcg(2024)
    calls = []  # (name, zero-arg launcher, output tensor)
    for m, n, k in ((8, 11008, 4096), (32, 11008, 4096), (8, 64, 16384), (48, 11008, 4096)):  # 48: two passes
        x, w, b = _up(dev, rng.normal((m, k))), _up(dev, rng.normal((n, k), 0.0, 0.05)), _up(dev, rng.normal((n,)))
        y = Tensor.empty([m, n], dev)
        calls.append((f"linear wT m={m} n={n} k={k}",
                      lambda m=m, n=n, k=k, x=x, w=w, b=b, y=y: lib.bch_sgemm_ex(
                          dev.ctx, 1, m, n, k, C.c_void_p(x.ptr), k, C.c_void_p(w.ptr), k, C.c_void_p(b.ptr),
                          N.BCH_ACT_GELU, C.c_void_p(y.ptr), n), y))
    for m, n, k in ((8, 11008, 4096), (48, 11008, 4096)):  # 48: the 64-row skinny kernel
        xa, wa = _up(dev, rng.normal((m, k))), _up(dev, rng.normal((k, n), 0.0, 0.02))
        ya = Tensor.empty([m, n], dev)
        calls.append((f"skinny m={m}", lambda m=m, n=n, k=k, xa=xa, wa=wa, ya=ya: lib.bch_sgemm(
            dev.ctx, m, n, k, C.c_void_p(xa.ptr), k, C.c_void_p(wa.ptr), n, C.c_void_p(ya.ptr), n), ya))
    for m2, n2, k2 in ((3072, 3072, 1024), (1024, 1024, 4096), (512, 512, 512)):  # hybrid, split-K, 64x64 tiles
        xg, wg = _up(dev, rng.uniform((m2, k2))), _up(dev, rng.uniform((k2, n2)))
        yg = Tensor.empty([m2, n2], dev)
        calls.append((f"sgemm {m2}x{n2}x{k2} ({lib.bch_sgemm_kernel_name(m2, n2, k2).decode()})",
                      lambda m2=m2, n2=n2, k2=k2, xg=xg, wg=wg, yg=yg: lib.bch_sgemm(
                          dev.ctx, m2, n2, k2, C.c_void_p(xg.ptr), k2, C.c_void_p(wg.ptr), n2, C.c_void_p(yg.ptr), n2),
                      yg))
    rows, cols = 512, 2048
    sx = _up(dev, rng.normal((rows, cols), 0.0, 3.0))
    sy = Tensor.empty([rows, cols], dev)
    calls.append(("softmax rows", lambda: lib.bch_softmax_rows(dev.ctx, rows, cols, C.c_void_p(sx.ptr),
                                                                C.c_void_p(sy.ptr)), sy))
    B, H, S, D = 1, 4, 256, 128
    q, kk, v = (_up(dev, rng.normal((B, H, S, D))) for _ in range(3))
    o = Tensor.empty([B, H, S, D], dev)
    calls.append(("sdpa causal", lambda: lib.bch_sdpa_fwd(dev.ctx, B, H, S, S, D, C.c_float(D ** -0.5), 1,
                                                           C.c_void_p(q.ptr), C.c_void_p(kk.ptr), C.c_void_p(v.ptr),
                                                           C.c_void_p(o.ptr)), o))

    # eager results (these calls also size the workspace, so the capture allocates nothing)
    want = []
    for name, run, out in calls:
        with dev._lock:
            dev.check(run(), name)
        want.append(out.to_numpy())

    graph, exe = C.c_void_p(), C.c_void_p()
    with dev._lock:
        assert hip.hipStreamBeginCapture(stream, CAPTURE_RELAXED) == 0
        try:
            for name, run, _ in calls:
                dev.check(run(), name + " (captured)")
        finally:
            assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
    try:
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        nan_fill = [np.full(out.to_numpy().shape, np.nan, np.float32) for _, _, out in calls]
        for rep in range(4):
            for (_, _, out), fill in zip(calls, nan_fill):
                dev.upload(out.ptr, fill)
            with dev._lock:
                assert hip.hipGraphLaunch(exe, stream) == 0
            dev.sync()
            for (name, _, out), ref in zip(calls, want):
                assert np.array_equal(out.to_numpy(), ref), (rep, name)
            # eager calls between the replays: the same workspace, flags and outputs
            for (name, run, out), ref in zip(calls, want):
                with dev._lock:
                    dev.check(run(), name)
                assert np.array_equal(out.to_numpy(), ref), (rep, name, "eager")
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)


class _FreshCtx:
    """A context of its own (its workspace starts empty), destroyed on exit."""

    def __init__(self, dev):
        self.lib = dev._lib
        self.ctx = C.c_void_p()
        assert self.lib.bch_ctx_create(0, None, C.byref(self.ctx)) == N.BCH_OK
        self.stream = C.c_void_p()
        assert self.lib.bch_ctx_stream(self.ctx, C.byref(self.stream)) == N.BCH_OK

    def ws_bytes(self) -> int:
        n = C.c_size_t()
        assert self.lib.bch_ctx_workspace_bytes(self.ctx, C.byref(n)) == N.BCH_OK
        return n.value

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.lib.bch_ctx_destroy(self.ctx)


def test_capture_that_would_grow_the_workspace_is_refused(dev):
    """A fresh context whose first call (split-K GEMM, needs a workspace) is made under
    capture: BCH_E_UNSUPPORTED with the reason, nothing recorded, no allocation; the same
    call then works eagerly, captures and replays.  After an eager call grows the
    workspace, the graph captured before still replays correctly: the old workspace it
    reads is kept alive, not freed."""
    _say("capture refusal, then capture after an eager call, then growth after the capture")
    hip = _hip()
    rng = O.Lcg(77)
    m = n = k = 1024  # split-K: slices in the workspace, then the reduce
    a, b = _up(dev, rng.uniform((m, k))), _up(dev, rng.uniform((k, n)))
    c = Tensor.empty([m, n], dev)
    want = a.to_numpy().astype(np.float64) @ b.to_numpy().astype(np.float64)
    with _FreshCtx(dev) as f:
        lib = f.lib
        call = lambda: lib.bch_sgemm(f.ctx, m, n, k, C.c_void_p(a.ptr), k, C.c_void_p(b.ptr), n,
                                     C.c_void_p(c.ptr), n)
        assert f.ws_bytes() == 0
        graph = C.c_void_p()
        assert hip.hipStreamBeginCapture(f.stream, CAPTURE_RELAXED) == 0
        st = call()
        assert hip.hipStreamEndCapture(f.stream, C.byref(graph)) == 0
        assert st == N.BCH_E_UNSUPPORTED
        assert "captured" in N.last_error(f.ctx) and "bch_ctx_reserve" in N.last_error(f.ctx)
        nodes = C.c_size_t()
        assert hip.hipGraphGetNodes(graph, None, C.byref(nodes)) == 0 and nodes.value == 0
        hip.hipGraphDestroy(graph)
        assert f.ws_bytes() == 0  # refused before any allocation
        assert call() == N.BCH_OK and lib.bch_sync(f.ctx) == N.BCH_OK  # eager: sizes the workspace
        ws0 = f.ws_bytes()
        assert ws0 > 0
        assert O.max_rel_err(c.to_numpy(), want) <= 1e-4
        eager = c.to_numpy()
        graph, exe = C.c_void_p(), C.c_void_p()
        assert hip.hipStreamBeginCapture(f.stream, CAPTURE_RELAXED) == 0
        st = call()
        assert hip.hipStreamEndCapture(f.stream, C.byref(graph)) == 0
        assert st == N.BCH_OK
        try:
            assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
            # an eager call that needs a larger workspace replaces it after the capture
            assert lib.bch_ctx_reserve(f.ctx, 4 * ws0) == N.BCH_OK
            assert f.ws_bytes() >= 4 * ws0
            for rep in range(3):
                dev.upload(c.ptr, np.full((m, n), np.nan, np.float32))
                assert hip.hipGraphLaunch(exe, f.stream) == 0
                assert lib.bch_sync(f.ctx) == N.BCH_OK
                assert np.array_equal(c.to_numpy(), eager), rep
        finally:
            if exe.value:
                hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)


def test_reserve_then_capture_allocates_nothing(dev):
    """bch_ctx_reserve sizes a fresh context's workspace up front; calls captured in global
    mode (where an allocation fails) then record only kernels, and replays match the eager
    results of another context."""
    _say("reserve, then global-mode capture of split-K GEMM, softmax over few long rows, wide attention")
    hip = _hip()
    rng = O.Lcg(78)
    a, b = _up(dev, rng.uniform((1024, 4096))), _up(dev, rng.uniform((4096, 1024)))
    c, c_ref = Tensor.empty([1024, 1024], dev), Tensor.empty([1024, 1024], dev)
    x = _up(dev, rng.normal((1, 1 << 20), 0.0, 3.0))
    y, y_ref = Tensor.empty([1, 1 << 20], dev), Tensor.empty([1, 1 << 20], dev)
    B, H, S, D = 1, 2, 96, 320
    q, kk, v = (_up(dev, rng.normal((B, H, S, D))) for _ in range(3))
    o, o_ref = Tensor.empty([B, H, S, D], dev), Tensor.empty([B, H, S, D], dev)
    P = lambda t: C.c_void_p(t.ptr)
    calls = [
        lambda ctx, out: dev._lib.bch_sgemm(ctx, 1024, 1024, 4096, P(a), 4096, P(b), 1024, P(out), 1024),
        lambda ctx, out: dev._lib.bch_softmax_rows(ctx, 1, 1 << 20, P(x), P(out)),
        lambda ctx, out: dev._lib.bch_sdpa_fwd(ctx, B, H, S, S, D, C.c_float(D ** -0.5), 1, P(q), P(kk), P(v),
                                               P(out)),
    ]
    outs, refs = [c, y, o], [c_ref, y_ref, o_ref]
    with dev._lock:
        for call, r in zip(calls, refs):
            dev.check(call(dev.ctx, r), "eager reference")
    dev.sync()
    with _FreshCtx(dev) as f:
        assert f.lib.bch_ctx_reserve(f.ctx, 64 << 20) == N.BCH_OK and f.lib.bch_sync(f.ctx) == N.BCH_OK
        ws = f.ws_bytes()
        assert ws >= 64 << 20
        graph, exe = C.c_void_p(), C.c_void_p()
        assert hip.hipStreamBeginCapture(f.stream, CAPTURE_GLOBAL) == 0
        sts = [call(f.ctx, out) for call, out in zip(calls, outs)]
        assert hip.hipStreamEndCapture(f.stream, C.byref(graph)) == 0
        assert sts == [N.BCH_OK] * 3, [N.last_error(f.ctx)]
        assert f.ws_bytes() == ws
        try:
            assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
            for rep in range(3):
                for out in outs:
                    dev.upload(out.ptr, np.full(out.shape(), np.nan, np.float32))
                assert hip.hipGraphLaunch(exe, f.stream) == 0
                assert f.lib.bch_sync(f.ctx) == N.BCH_OK
                for out, r in zip(outs, refs):
                    assert np.array_equal(out.to_numpy(), r.to_numpy()), rep
        finally:
            if exe.value:
                hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)
