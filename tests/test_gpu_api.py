"""Host API on the GPU: seeded device fills vs the oracle's generators, the
reference tests' error paths, and allocation-failure injection."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

from barracuda_amd import LcgStream, Tensor
from barracuda_amd.error import ShapeMismatch
from oracle import bc_oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("seed", [0, 2, 12345])
def test_device_uniform_fill_is_bit_exact(dev, seed):
    _say(f"fill_uniform seed {seed}")
    s = LcgStream(seed, dev)
    a = s.uniform([1000, 37]).to_numpy()
    b = s.uniform([3, 5], 0.0, 1.0).to_numpy()
    r = O.Lcg(seed)
    assert np.array_equal(a, r.uniform((1000, 37)))
    assert np.array_equal(b, r.uniform((3, 5), 0.0, 1.0))
    assert s.state.value == r.state.value


@pytest.mark.parametrize("seed,sigma", [(1, 3.0), (3, 0.02), (4, 1.0)])
def test_device_normal_fill_matches(dev, seed, sigma):
    _say(f"fill_normal seed {seed} sigma {sigma}")
    s = LcgStream(seed, dev)
    x = s.normal([4099 * 3], 0.0, sigma).to_numpy()
    y = s.normal([17]).to_numpy()
    r = O.Lcg(seed)
    rx, ry = r.normal(4099 * 3, 0.0, sigma), r.normal(17)
    # device log/cos (f64) vs host libm: equal after rounding to f32, or 1 ulp apart
    ulps = np.abs(x.view(np.int32).astype(np.int64) - rx.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.999
    assert np.array_equal(y.view(np.int32) // 2, ry.view(np.int32) // 2) or \
        np.abs(y.view(np.int32).astype(np.int64) - ry.view(np.int32)).max() <= 1
    assert s.state.value == r.state.value


def test_fault_injection_shape_error_message(dev):
    # T/fault_injection.rs:29-60: a mismatched matmul returns an error that
    # names shape/dimension/mismatch, and the device stays usable
    a = Tensor.from_data(np.ones(6, np.float32), [2, 3], dev)
    b = Tensor.from_data(np.ones(8, np.float32), [4, 2], dev)
    with pytest.raises(ShapeMismatch) as e:
        a.matmul(b)
    msg = str(e.value).lower()
    assert any(w in msg for w in ("shape", "dimension", "mismatch"))
    c = Tensor.from_data(np.ones(6, np.float32), [3, 2], dev)
    assert np.array_equal(a.matmul(c).to_vec(), np.full(4, 3.0, np.float32))


def test_alloc_failure_injection_maps_to_out_of_memory():
    _say("alloc failure injection (child process)")
    code = (
        "import numpy as np\n"
        "from barracuda_amd import Tensor, OutOfMemory, get_device\n"
        "d = get_device()\n"
        "try:\n"
        "    Tensor.from_data(np.ones(4, np.float32), [4], d)\n"
        "    print('NO-ERROR')\n"
        "except OutOfMemory as e:\n"
        "    print('OOM', e)\n")
    env = dict(os.environ, BARRACUDA_HIP_FAIL_ALLOC="1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=root, capture_output=True, text=True,
                       timeout=120)
    assert "OOM" in r.stdout, r.stdout + r.stderr
    assert "injected" in r.stdout


def test_device_copy(dev):
    _say("bch_copy aligned / unaligned")
    import ctypes as C
    x = O.Lcg(8).uniform(100003)
    src = Tensor.from_data(x, [100003], dev)
    dst = Tensor.empty([100003], dev)
    dev.check(dev._lib.bch_copy(dev.ctx, C.c_void_p(dst.ptr), C.c_void_p(src.ptr), 4 * 100000), "copy")
    got = dst.to_vec()
    assert np.array_equal(got[:100000], x[:100000])
    dst2 = Tensor.empty([100003], dev)
    dev.check(dev._lib.bch_copy(dev.ctx, C.c_void_p(dst2.ptr + 4), C.c_void_p(src.ptr + 8), 4 * 99990 + 3),
              "copy")
    got2 = dst2.to_vec()
    assert np.array_equal(got2[1:99991], x[2:99992])
    assert got2.view(np.uint8)[4 + 4 * 99990: 4 + 4 * 99990 + 3].tolist() == \
        x.view(np.uint8)[8 + 4 * 99990: 8 + 4 * 99990 + 3].tolist()


def test_device_copy_runs_and_streaming_path(dev):
    """16-byte copies: sizes that end inside a wave's run and the >= 64 MB
    non-temporal path; the bytes after the copied range stay untouched."""
    import ctypes as C
    for n in (4, 4100, 4 * 1024 * 7 + 12, (64 << 20) // 4 + 4 * 333):
        _say(f"bch_copy {4 * n} bytes")
        x = O.Lcg(n).uniform(n)
        src = Tensor.from_data(x, [n], dev)
        dst = Tensor.from_data(np.full(n + 8, -7.0, np.float32), [n + 8], dev)
        dev.check(dev._lib.bch_copy(dev.ctx, C.c_void_p(dst.ptr), C.c_void_p(src.ptr), 4 * n), "copy")
        got = dst.to_vec()
        assert np.array_equal(got[:n], x) and np.all(got[n:] == -7.0)


def test_pool_hands_freed_blocks_back(dev):
    """bch_free parks a block for the next bch_alloc of its size class (powers of two from
    256 bytes to 64 MiB, then multiples of 2 MiB), as the reference's buffer pool does."""
    import ctypes as C
    _say("pool: freed blocks come back by size class")
    lib, ctx = dev._lib, dev.ctx

    def alloc(nbytes):
        p = C.c_void_p()
        dev.check(lib.bch_alloc(ctx, nbytes, C.byref(p)), "alloc")
        return p.value

    def free(p):
        dev.check(lib.bch_free(ctx, C.c_void_p(p)), "free")

    p1 = alloc(1000)
    free(p1)
    assert alloc(900) == p1            # the same 1 KiB class
    p2 = alloc(3000)                   # a 4 KiB class: a new block
    assert p2 != p1
    free(p1)
    free(p2)
    big = alloc((100 << 20) + 5)       # above 64 MiB: multiples of 2 MiB
    free(big)
    assert alloc((101 << 20) + 7) == big
    free(big)


def test_pool_reuse_is_ordered_on_the_stream(dev):
    """A block freed while queued copies still read it, taken back at once by bch_alloc and
    overwritten by an upload: the copies see the old contents, because the upload queues
    behind them on the context's stream (bch_free does not wait)."""
    import ctypes as C
    _say("pool: reuse is ordered behind the work that reads the block")
    lib, ctx = dev._lib, dev.ctx
    n = (256 << 20) // 4
    x = O.Lcg(77).uniform(n)
    p = C.c_void_p()
    dev.check(lib.bch_alloc(ctx, 4 * n, C.byref(p)), "alloc")
    src = p.value
    dev.check(lib.bch_upload(ctx, C.c_void_p(src), x.ctypes.data_as(C.c_void_p), 4 * n), "upload")
    dsts = [Tensor.empty([n], dev) for _ in range(4)]
    for d in dsts:  # ~0.35 ms of copies queued that read the block
        dev.check(lib.bch_copy(ctx, C.c_void_p(d.ptr), C.c_void_p(src), 4 * n), "copy")
    dev.check(lib.bch_free(ctx, C.c_void_p(src)), "free")
    q = C.c_void_p()
    dev.check(lib.bch_alloc(ctx, 4 * n, C.byref(q)), "alloc")
    assert q.value == src
    zeros = np.zeros(n, np.float32)
    dev.check(lib.bch_upload(ctx, q, zeros.ctypes.data_as(C.c_void_p), 4 * n), "upload")
    for d in dsts:
        assert np.array_equal(d.to_vec(), x)
    dev.check(lib.bch_free(ctx, q), "free")


def test_pool_recycles_tensor_outputs(dev):
    """A loop of ops on fresh output tensors reuses the same device memory once the previous
    results are dropped (no allocation per op in steady state)."""
    _say("pool: tensor outputs recycled")
    a = Tensor.from_data(O.Lcg(5).uniform((256, 256)), [256, 256], dev)
    seen = set()
    for i in range(6):
        c = a.matmul(a)
        seen.add(c.ptr)
        del c
    assert len(seen) <= 2, seen


def test_two_contexts_from_two_threads():
    """Two contexts on the device, driven from two threads at once: the
    per-device launch set-up (dynamic-LDS limits) is shared and locked, and
    each context's results stay its own."""
    import threading
    from barracuda_amd import HipDevice
    from oracle import bc_oracle as O
    print("two contexts, two threads", flush=True)
    rng = O.Lcg(31)
    a, b = rng.uniform((512, 512)), rng.uniform((512, 512))
    x, w = rng.normal((8, 1024)), rng.normal((1024, 2048), 0.0, 0.02)
    q = rng.normal((1, 4, 256, 128))
    want_mm, want_sk = O.matmul_f64(a, b), O.matmul_f64(x, w)
    want_at = O.sdpa_f64(q, q, q, True)
    errs = []

    def work(seed):
        try:
            d = HipDevice(0)
            for _ in range(3):
                c = Tensor.from_data(a, [512, 512], d).matmul(Tensor.from_data(b, [512, 512], d)).to_numpy()
                y = Tensor.from_data(x, [8, 1024], d).matmul(Tensor.from_data(w, [1024, 2048], d)).to_numpy()
                tq = Tensor.from_data(q, list(q.shape), d)
                o = tq.causal_attention(tq, tq).to_numpy()
                errs.append(max(O.max_rel_err(c, want_mm), O.max_rel_err(y, want_sk), O.max_rel_err(o, want_at)))
            d.close()
        except Exception as e:  # reported below
            errs.append(e)

    ts = [threading.Thread(target=work, args=(s,)) for s in (1, 2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert len(errs) == 6, errs
    assert all(isinstance(e, float) and e <= 1e-4 for e in errs), errs


@pytest.mark.parametrize("hip_error", [700, 719])  # hipErrorIllegalAddress, hipErrorLaunchFailure
def test_device_lost_injection_is_sticky(monkeypatch, hip_error):
    """A context-fatal HIP error (injected on the host: no kernel runs)
    becomes DeviceLost, is_lost() turns true, and every later device call on
    that context fails the same way (WgpuDevice::poll_safe's lost flag,
    device/wgpu_device/submission.rs:23-71; GpuBackend::is_lost, device/
    backend.rs:256).  A fresh context works."""
    _say(f"device-lost injection, hipError {hip_error}")
    from barracuda_amd import DeviceLost, HipDevice
    monkeypatch.setenv("BARRACUDA_HIP_INJECT_HIP_ERROR", str(hip_error))
    d = HipDevice(0)
    monkeypatch.delenv("BARRACUDA_HIP_INJECT_HIP_ERROR")
    assert not d.is_lost()
    with pytest.raises(DeviceLost, match=str(hip_error)):
        d.alloc(1024)
    assert d.is_lost()
    with pytest.raises(DeviceLost, match="device lost"):
        d.sync()
    with pytest.raises(DeviceLost):
        Tensor.from_data(np.ones(4, np.float32), [4], d)
    assert d.is_lost()
    d.close()
    d2 = HipDevice(0)
    assert not d2.is_lost()
    t = Tensor.from_data(np.arange(4, dtype=np.float32), [4], d2)
    assert np.array_equal(t.to_vec(), np.arange(4, dtype=np.float32))
    d2.close()


@pytest.mark.parametrize("hip_error,kind", [(2, "OutOfMemory"), (701, "ExecutionError"), (1, "DeviceError")])
def test_injected_recoverable_errors_keep_the_context(monkeypatch, hip_error, kind):
    """hipErrorOutOfMemory, hipErrorLaunchOutOfResources and
    hipErrorInvalidValue map to OutOfMemory, ExecutionError and Device; none
    marks the context lost, and the next call succeeds."""
    _say(f"recoverable injection, hipError {hip_error}")
    import barracuda_amd as B
    monkeypatch.setenv("BARRACUDA_HIP_INJECT_HIP_ERROR", str(hip_error))
    d = B.HipDevice(0)
    monkeypatch.delenv("BARRACUDA_HIP_INJECT_HIP_ERROR")
    with pytest.raises(getattr(B, kind)) as e:
        d.sync()
    assert not isinstance(e.value, B.DeviceLost)
    assert not d.is_lost()
    d.sync()
    t = Tensor.from_data(np.ones(8, np.float32), [2, 4], d)
    assert np.array_equal(t.to_vec(), np.ones(8, np.float32))
    d.close()


def test_ring_combine_timeout_is_reported(monkeypatch):
    """The [out, in] decode GEMM combines split-k blocks in its kernel with a bounded wait.
    BARRACUDA_HIP_RING_SPIN=0 (read at context creation) makes every owner give up at once,
    with every kernel still exiting normally: the outputs it could not combine are NaN, and the
    context reports DeviceLost at its next synchronisation and on every later call instead of
    returning NaN silently.  Another context computes the same call correctly."""
    _say("ring combine timeout forced from the host")
    import ctypes as C
    from barracuda_amd import DeviceLost, HipDevice
    m, n, k = 16, 11008, 4096  # 8 < m <= 32: the ring kernel with split groups
    good = HipDevice(0)
    rng = O.Lcg(616)
    x, w = rng.normal((m, k)), rng.normal((n, k), 0.0, 0.02)
    tx, tw = Tensor.from_data(x, [m, k], good), Tensor.from_data(w, [n, k], good)
    ty = Tensor.from_data(np.zeros((m, n), np.float32), [m, n], good)
    monkeypatch.setenv("BARRACUDA_HIP_RING_SPIN", "0")
    d = HipDevice(0)
    monkeypatch.delenv("BARRACUDA_HIP_RING_SPIN")
    lib = d._lib
    st = lib.bch_sgemm_ex(d.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr), k, None, 0,
                          C.c_void_p(ty.ptr), n)
    assert st == 0
    with pytest.raises(DeviceLost, match="split-k combine timed out"):
        d.sync()
    assert d.is_lost()
    with pytest.raises(DeviceLost):
        d.sync()
    got = ty.to_numpy()  # through the healthy context
    assert np.isnan(got).any()
    d.close()
    good.check(lib.bch_sgemm_ex(good.ctx, 1, m, n, k, C.c_void_p(tx.ptr), k, C.c_void_p(tw.ptr), k, None, 0,
                                C.c_void_p(ty.ptr), n), "sgemm_ex")
    assert O.max_rel_err(ty.to_numpy(), O.matmul_f64(x, np.ascontiguousarray(w.T))) <= 1e-4
    assert not good.is_lost()
    del tx, tw, ty
    good.close()
