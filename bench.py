#!/usr/bin/env python3
"""Benchmark of the MI355X hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

Headline (`value`): f32 GEMM M=N=K=4096 in TFLOP/s:
one step = one bch_sgemm launch over inputs already resident in HBM (seeded
U[-1,1) from the reference's LCG, seed 2, generated on the device).  The
other configurations (row softmax, skinny GEMM, batched GEMM, fused
attention) are measured in the same run and reported under "extra".

Timing: HIP events recorded on the library's own stream (bch_event_*) give
the average kernel duration used for `roofline`; the wall clock around
exactly K launches, bracketed by bch_sync on both sides, gives ms_per_step.
`cpu_baseline` is the reference's CPU matmul (execute_matmul_cpu, restated
in oracle/) timed on this host on a bounded row sample.
"""
from __future__ import annotations

import argparse
import ctypes as C

import numpy as np
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix, published
FP64_MFMA_PEAK_TFLOPS = 78.6   # MI355X dense FP64 matrix, published
PROFILES = ROOT / "profiles"
# Before every timed region's warmup launches, another kernel keeps the GPU
# busy for this long (the clock settle, ClockWarmer).
SETTLE_MS = 60.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class ClockWarmer:
    """Brings the clocks to steady state before a timed region with a kernel
    other than the one about to be timed: the 4096^3 GEMM with B given as
    [n][k] (bch_sgemm_ex, transb, no epilogue), a different kernel
    instantiation from every workload here.  From idle the clocks take ~25
    ms of full load to settle (measured on the box: 4096^3 launches go
    1100-1190 us -> 940-945 us over the first ~25 launches), and each
    workload starts after host-side set-up has left the GPU idle.  Warming
    with another kernel keeps the timed kernel's own launches (W warmup + K
    timed) all at steady clocks, so a profiler's per-kernel average over the
    run agrees with the HIP-event average of the timed launches."""

    N = 4096

    def __init__(self, dev):
        from barracuda_amd import LcgStream, Tensor
        self.dev = dev
        s = LcgStream(17, dev)
        self._a, self._b = s.uniform([self.N, self.N]), s.uniform([self.N, self.N])
        self._c = Tensor.empty([self.N, self.N], dev)

    def run(self, ms: float) -> None:
        dev, lib, n = self.dev, self.dev._lib, self.N
        pa, pb, pc = C.c_void_p(self._a.ptr), C.c_void_p(self._b.ptr), C.c_void_p(self._c.ptr)
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < ms:
            for _ in range(4):
                dev.check(lib.bch_sgemm_ex(dev.ctx, 1, n, n, n, pa, n, pb, n, None, 0, pc, n), "clock warm-up")
            dev.sync()


class Timer:
    """HIP events on the context's stream + wall clock around K launches.

    Before the W warmup launches, the ClockWarmer keeps the GPU busy with
    another kernel for `warm_ms` (the clock settle)."""

    def __init__(self, dev, warm_ms: float = 0.0, warmer: ClockWarmer | None = None):
        self.dev = dev
        self.warm_ms = warm_ms
        self.warmer = warmer if warmer is not None or warm_ms <= 0 else ClockWarmer(dev)
        lib = dev._lib
        self.e0, self.e1 = C.c_void_p(), C.c_void_p()
        dev.check(lib.bch_event_create(dev.ctx, C.byref(self.e0)), "event")
        dev.check(lib.bch_event_create(dev.ctx, C.byref(self.e1)), "event")

    def run(self, fn, steps: int, warmup: int):
        lib, dev = self.dev._lib, self.dev
        if self.warmer is not None:
            self.warmer.run(self.warm_ms)
        for _ in range(warmup):
            dev.check(fn(0) or 0, "bench warmup launch")
        dev.sync()
        t0 = time.perf_counter()
        dev.check(lib.bch_event_record(dev.ctx, self.e0), "event")
        failed = 0
        for i in range(steps):
            failed = failed or fn(i) or 0
        dev.check(lib.bch_event_record(dev.ctx, self.e1), "event")
        dev.check(failed, "bench launch")
        dev.sync()
        t1 = time.perf_counter()
        ms = C.c_float()
        dev.check(lib.bch_event_elapsed_ms(self.e0, self.e1, C.byref(ms)), "event")
        return (t1 - t0) * 1e3 / steps, ms.value / steps  # wall ms/step, event ms/launch


def load_traffic(key: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summaries
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    f = PROFILES / "traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return d.get(key, {}).get("bytes_per_launch")
    except Exception:
        return None


def bench_gemm(dev, steps, warmup, warmer=None):
    from barracuda_amd import LcgStream
    lib = dev._lib
    n = 4096
    s = LcgStream(2, dev)
    a, b = s.uniform([n, n]), s.uniform([n, n])
    from barracuda_amd import Tensor
    c = Tensor.empty([n, n], dev)
    ctx, pa, pb, pc = dev.ctx, C.c_void_p(a.ptr), C.c_void_p(b.ptr), C.c_void_p(c.ptr)

    def step(_i):
        st = lib.bch_sgemm(ctx, n, n, n, pa, n, pb, n, pc, n)
        if st:
            dev.check(st, "sgemm")

    # The same clock settle as every other workload: from idle, the clocks
    # take ~25 ms of full load to reach steady state, so W warmup launches
    # alone (the driver passes W = 5) would time the ramp.
    wall_ms, ev_ms = Timer(dev, warm_ms=SETTLE_MS, warmer=warmer).run(step, steps, warmup)
    flops = 2.0 * n ** 3
    return {"wall_ms": wall_ms, "kernel_ms": ev_ms, "flops": flops,
            "kernel": lib.bch_sgemm_kernel_name(n, n, n).decode()}, (a, b, c)


WORKLOADS = ("softmax", "skinny", "batched", "sdpa", "linear", "dgemm", "norm", "attn64", "copy")


def bench_extra(dev, reps: int = 20, only=None, warmer=None, skinny_n: int = 11008):
    """The other BASELINE configs, each timed over `reps` launches."""
    from barracuda_amd import LcgStream, Tensor
    lib, ctx = dev._lib, dev.ctx
    T = Timer(dev, warm_ms=SETTLE_MS, warmer=warmer)
    out = {}
    want = set(only) if only else set(WORKLOADS) - {"copy"}

    if "copy" in want:
        # known-traffic reference: 512 MiB read + 512 MiB written
        nb = 512 << 20
        src = LcgStream(9, dev).uniform([nb // 4])
        dst = Tensor.empty([nb // 4], dev)
        ps, pd = C.c_void_p(src.ptr), C.c_void_p(dst.ptr)
        wall, ev = T.run(lambda i: lib.bch_copy(ctx, pd, ps, nb), reps, 3)
        out["copy_512MiB"] = {"GB/s": 2 * nb / (ev * 1e-3) / 1e9, "us": ev * 1e3, "bytes_per_launch": 2 * nb,
                              "hbm_frac": 2 * nb / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
        del src, dst
    if "softmax" in want:
        out.update(_bench_softmax(dev, T, reps))
    if "skinny" in want:
        out.update(_bench_skinny(dev, T, reps, skinny_n))
    if "batched" in want:
        out.update(_bench_batched(dev, T, reps))
    if "sdpa" in want:
        out.update(_bench_sdpa(dev, T, reps))
    if "linear" in want:
        out.update(_bench_linear(dev, T, reps))
    if "dgemm" in want:
        out.update(_bench_dgemm(dev, T, reps))
    if "norm" in want:
        out.update(_bench_norm(dev, T, reps))
    if "attn64" in want:
        out.update(_bench_attn64(dev, T, reps))
    return out


def _bench_attn64(dev, T, reps):
    """The f64 route of the ml.attention handler (ml/forward.rs:121-150):
    its row softmax alone over [32768 x 2048] f64 (one read + one write,
    16 B per element, HBM-bound), and the whole computation at seq_q = seq_k
    = 2048, d_k = d_v = 128 (Q K^T and P V on bch_dgemm, the softmax between
    them), operands resident in HBM."""
    from barracuda_amd import F64Buffer
    lib, ctx = dev._lib, dev.ctx
    out = {}
    rng = np.random.default_rng(5)
    rows, cols = 32768, 2048
    x = F64Buffer(dev, rows * cols).upload(rng.standard_normal(rows * cols) * 3.0)
    y = F64Buffer(dev, rows * cols)
    px, py = C.c_void_p(x.ptr), C.c_void_p(y.ptr)
    nbytes = 2 * 8 * rows * cols
    wall, ev = T.run(lambda i: lib.bch_softmax_rows_f64(ctx, rows, cols, px, py), reps, 3)
    out["softmax_f64_32768x2048"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3, "bytes_per_launch": nbytes,
                                     "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                     "kernel": lib.bch_softmax_rows_f64_kernel_name(rows, cols, px, py).decode()}
    del x, y
    s, d = 2048, 128
    q, k, v = (F64Buffer(dev, s * d).upload(rng.standard_normal(s * d)) for _ in range(3))
    sc, o = F64Buffer(dev, s * s), F64Buffer(dev, s * d)
    pq, pk, pv, ps, po = (C.c_void_p(t.ptr) for t in (q, k, v, sc, o))
    scale = 1.0 / float(np.sqrt(d))

    def step(i):
        st = lib.bch_dgemm(ctx, 0, 1, 1, s, s, d, scale, pq, d, s * d, pk, d, s * d, 0.0, ps, s, s * s)
        st = st or lib.bch_softmax_rows_f64(ctx, s, s, ps, ps)
        return st or lib.bch_dgemm(ctx, 0, 0, 1, s, d, s, 1.0, ps, s, s * s, pv, d, s * d, 0.0, po, d, s * d)
    wall, ev = T.run(step, reps, 3)
    fl = 2.0 * 2 * s * s * d
    out["ml_attention_f64_2048x2048x128"] = {"us": ev * 1e3, "TFLOP/s": fl / (ev * 1e-3) / 1e12,
                                             "fp64_mfma_frac": fl / (ev * 1e-3) / 1e12 / FP64_MFMA_PEAK_TFLOPS}
    return out


def _bench_norm(dev, T, reps):
    """The steps either side of the path (TensorSession::layer_norm and
    ::gelu, session/mod.rs:349-398) at the softmax config's size: layer norm
    of [65536 x 2048] (one read + one write, 8 B per element) and GELU over
    the same 2^27 elements; the session's head_split / head_concat at the
    attention config's shape.  All HBM-bound."""
    from barracuda_amd import LcgStream, Tensor
    from barracuda_amd import _native as N
    lib, ctx = dev._lib, dev.ctx
    out = {}
    rows, cols = 65536, 2048
    x = LcgStream(1, dev).normal([rows, cols], 0.0, 3.0)
    y = Tensor.empty([rows, cols], dev)
    px, py = C.c_void_p(x.ptr), C.c_void_p(y.ptr)
    nbytes = 2 * 4 * rows * cols
    wall, ev = T.run(lambda i: lib.bch_layer_norm(ctx, rows, cols, 1e-5, px, py), reps, 3)
    out["layer_norm_65536x2048"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3, "bytes_per_launch": nbytes,
                                    "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                    "kernel": lib.bch_layer_norm_kernel_name(rows, cols, px, py).decode()}
    n = rows * cols
    wall, ev = T.run(lambda i: lib.bch_elementwise(ctx, N.BCH_EW_GELU, n, px, None, None, 0.0, py), reps, 3)
    out["gelu_2^27"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3, "bytes_per_launch": nbytes,
                        "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
    del x, y
    # TensorSession::head_split / head_concat (session/mod.rs:423-480) at the attention
    # config's shape: [4, 2048, 32*128] <-> [4, 32, 2048, 128], a copy (8 B per element)
    B, S, H, D = 4, 2048, 32, 128
    n = B * S * H * D
    x = LcgStream(3, dev).normal([n], 0.0, 1.0)
    y = Tensor.empty([n], dev)
    px, py = C.c_void_p(x.ptr), C.c_void_p(y.ptr)
    nbytes = 2 * 4 * n
    for name, fn in (("head_split", lib.bch_head_split), ("head_concat", lib.bch_head_concat)):
        wall, ev = T.run(lambda i: fn(ctx, B, S, H, D, px, py), reps, 3)
        out[f"{name}_4x2048x32x128"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3,
                                        "bytes_per_launch": nbytes,
                                        "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


def _bench_dgemm(dev, T, reps):
    """GemmF64 (ops/linalg/gemm_f64.rs) at 4096^3 on the FP64 matrix cores,
    operands resident in HBM."""
    from barracuda_amd import F64Buffer
    lib, ctx = dev._lib, dev.ctx
    n = 4096
    rng = np.random.default_rng(2)
    a = F64Buffer(dev, n * n).upload(rng.uniform(-1, 1, n * n))
    b = F64Buffer(dev, n * n).upload(rng.uniform(-1, 1, n * n))
    c = F64Buffer(dev, n * n)
    pa, pb, pc = C.c_void_p(a.ptr), C.c_void_p(b.ptr), C.c_void_p(c.ptr)
    wall, ev = T.run(lambda i: lib.bch_dgemm(ctx, 0, 0, 1, n, n, n, 1.0, pa, n, n * n, pb, n, n * n, 0.0, pc, n,
                                             n * n), max(5, reps // 2), 2)
    fl = 2.0 * n ** 3
    return {"dgemm_4096": {"TFLOP/s": fl / (ev * 1e-3) / 1e12, "ms": ev,
                           "fp64_mfma_frac": fl / (ev * 1e-3) / 1e12 / FP64_MFMA_PEAK_TFLOPS}}


def _bench_linear(dev, T, reps):
    """The linear layer of nn::fused_mlp at the GEMM config's size: y =
    relu(x W^T + b), W [out, in] = [4096, 4096], one launch (bias and ReLU in
    the GEMM epilogue)."""
    from barracuda_amd import LcgStream, Tensor
    from barracuda_amd import _native as N
    lib, ctx = dev._lib, dev.ctx
    n = 4096
    s = LcgStream(5, dev)
    x, w, b = s.uniform([n, n]), s.uniform([n, n]), s.uniform([n])
    y = Tensor.empty([n, n], dev)
    px, pw, pb, py = (C.c_void_p(t.ptr) for t in (x, w, b, y))
    wall, ev = T.run(lambda i: lib.bch_sgemm_ex(ctx, 1, n, n, n, px, n, pw, n, pb, N.BCH_ACT_RELU, py, n), reps, 3)
    fl = 2.0 * n ** 3
    out = {"linear_4096_wT_bias_relu": {"TFLOP/s": fl / (ev * 1e-3) / 1e12, "ms": ev,
                                        "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS}}
    wall, ev = T.run(lambda i: lib.bch_sgemm_ex(ctx, 1, n, n, n, px, n, pw, n, pb, N.BCH_ACT_GELU, py, n), reps, 3)
    out["linear_4096_wT_bias_gelu"] = {"TFLOP/s": fl / (ev * 1e-3) / 1e12, "ms": ev,
                                       "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS}
    del x, w, b, y
    # decode-sized layers with [out, in] weights (the skinny config's shape, W^T): HBM-bound
    K, Nn = 4096, 11008
    ws = [s.normal([Nn, K], 0.0, 0.02) for _ in range(3)]
    bias = s.normal([Nn])
    pws, pbias = [C.c_void_p(t.ptr) for t in ws], C.c_void_p(bias.ptr)
    for m in (1, 8, 32):
        xs, ys = s.normal([m, K]), Tensor.empty([m, Nn], dev)
        pxs, pys = C.c_void_p(xs.ptr), C.c_void_p(ys.ptr)
        wall, ev = T.run(lambda i: lib.bch_sgemm_ex(ctx, 1, m, Nn, K, pxs, K, pws[i % 3], K, pbias, N.BCH_ACT_RELU,
                                                    pys, Nn), reps, 3)
        nbytes = 4 * (K * Nn + m * K + m * Nn + Nn)
        out[f"linear_decode_wT_m{m}"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3,
                                         "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


def _bench_softmax(dev, T, reps):
    from barracuda_amd import LcgStream, Tensor
    lib, ctx = dev._lib, dev.ctx
    out = {}
    # config 2: row softmax [65536 x 2048], N(0,3), seed 1
    x = LcgStream(1, dev).normal([65536, 2048], 0.0, 3.0)
    y = Tensor.empty([65536, 2048], dev)
    px, py = C.c_void_p(x.ptr), C.c_void_p(y.ptr)
    wall, ev = T.run(lambda i: lib.bch_softmax_rows(ctx, 65536, 2048, px, py), reps, 3)
    nbytes = 2 * 4 * 65536 * 2048
    out["softmax_65536x2048"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "kernel_us": ev * 1e3,
                                 "bytes_per_launch": nbytes,
                                 "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                 "traffic": load_traffic("softmax_65536x2048")}
    # Tensor::softmax (global) over the same 2^27 elements as one row: the
    # split-row path, two passes (12 bytes per element of traffic at least)
    n = 65536 * 2048
    wall, ev = T.run(lambda i: lib.bch_softmax_rows(ctx, 1, n, px, py), reps, 3)
    out["softmax_global_2^27"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3,
                                  "bytes_per_call": nbytes, "traffic": load_traffic("softmax_global_2^27"),
                                  "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                  "hbm_frac_of_12B_floor": 1.5 * nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # softmax_dim over a middle axis of the same 2^27 elements: [64, 2048, 1024] (whole column
    # strips in registers, one read) and [1, 65536, 2048] (a chunked axis, read twice)
    for (o, a, inn), path in (((64, 2048, 1024), "column strips in registers"),
                              ((1, 65536, 2048), "chunked axis, whole-row passes: stats + merge + write")):
        wall, ev = T.run(lambda i: lib.bch_softmax_axis(ctx, o, a, inn, px, py), reps, 3)
        out[f"softmax_axis_{o}x{a}x{inn}"] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3,
                                              "bytes_per_call": nbytes, "path": path,
                                              "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


def _bench_skinny(dev, T, reps, N: int = 11008):
    from barracuda_amd import LcgStream, Tensor
    lib, ctx = dev._lib, dev.ctx
    out = {}
    # config 4: skinny GEMM M in {1, 8, 32}, K 4096, N 11008; X ~ N(0,1), W ~ N(0,0.02), seed 3.
    # Three weight copies (541 MB > the 256 MB Infinity Cache) are rotated.  A larger N
    # (--skinny-n, profiling only) lengthens each launch so that per-dispatch counter windows
    # are dominated by the kernel.
    K = 4096
    for m in (1, 8, 32):
        s = LcgStream(3, dev)
        xs = s.normal([m, K])
        ws = [s.normal([K, N], 0.0, 0.02) for _ in range(3)]
        ys = Tensor.empty([m, N], dev)
        pxs, pys = C.c_void_p(xs.ptr), C.c_void_p(ys.ptr)
        pws = [C.c_void_p(w.ptr) for w in ws]
        wall, ev = T.run(lambda i: lib.bch_sgemm(ctx, m, N, K, pxs, K, pws[i % 3], N, pys, N), reps, 3)
        nbytes = 4 * (K * N + m * K + m * N)
        out[f"skinny_m{m}" + ("" if N == 11008 else f"_n{N}")] = {"GB/s": nbytes / (ev * 1e-3) / 1e9, "us": ev * 1e3,
                               "bytes_per_call": nbytes,
                               "hbm_frac": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
                               "TFLOP/s": 2.0 * m * K * N / (ev * 1e-3) / 1e12,
                               "traffic": load_traffic(f"skinny_m{m}")}
        del xs, ws, ys
    return out


def _bench_batched(dev, T, reps):
    from barracuda_amd import LcgStream, Tensor
    lib, ctx = dev._lib, dev.ctx
    out = {}
    # config 3b: batched 16 x 1024^3, U[-1,1), seed 2
    s = LcgStream(2, dev)
    a, b = s.uniform([16, 1024, 1024]), s.uniform([16, 1024, 1024])
    c = Tensor.empty([16, 1024, 1024], dev)
    pa, pb, pc = C.c_void_p(a.ptr), C.c_void_p(b.ptr), C.c_void_p(c.ptr)
    mm = 1024 * 1024
    wall, ev = T.run(lambda i: lib.bch_sgemm_strided_batched(ctx, 16, 1024, 1024, 1024, pa, mm, pb, mm,
                                                              pc, mm), reps, 3)
    fl = 2.0 * 16 * 1024 ** 3
    out["batched_16x1024"] = {"TFLOP/s": fl / (ev * 1e-3) / 1e12, "ms": ev,
                              "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                              "traffic": load_traffic("sgemm_batched_16x1024")}
    del a, b, c
    # config 1's shape on the GPU, beside its CPU-path time in extra.cpu.matmul_256
    s0 = LcgStream(0, dev)
    a, b = s0.uniform([256, 256]), s0.uniform([256, 256])
    c = Tensor.empty([256, 256], dev)
    pa, pb, pc = C.c_void_p(a.ptr), C.c_void_p(b.ptr), C.c_void_p(c.ptr)
    wall, ev = T.run(lambda i: lib.bch_sgemm(ctx, 256, 256, 256, pa, 256, pb, 256, pc, 256), reps, 3)
    out["matmul_256"] = {"us": ev * 1e3, "GFLOP/s": 2.0 * 256 ** 3 / (ev * 1e-3) / 1e9,
                         "kernel": lib.bch_sgemm_kernel_name(256, 256, 256).decode()}
    del a, b, c
    # MatMul at shapes whose tiles do not come out in whole rounds of the CUs: the tile
    # choice, the hybrid plan (whole tiles + k-sliced leftover tiles), the mixed plan (whole
    # rounds of 256x256 tiles on the first columns / rows, then the rest), split-K and the
    # float4-guarded ragged loads, beside the headline's whole-round 4096^3
    shapes = {}
    for m, n, k in ((3072, 3072, 3072), (5120, 5120, 5120), (6144, 6144, 6144), (4096, 11008, 4096),
                    (11008, 4096, 4096), (4000, 4000, 4000), (1024, 1024, 1024)):
        s1 = LcgStream(m + n + k, dev)
        a, b = s1.uniform([m, k]), s1.uniform([k, n])
        c = Tensor.empty([m, n], dev)
        pa, pb, pc = C.c_void_p(a.ptr), C.c_void_p(b.ptr), C.c_void_p(c.ptr)
        wall, ev = T.run(lambda i, m=m, n=n, k=k: lib.bch_sgemm(ctx, m, n, k, pa, k, pb, n, pc, n), reps, 3)
        fl = 2.0 * m * n * k
        shapes[f"{m}x{n}x{k}"] = {"TFLOP/s": fl / (ev * 1e-3) / 1e12, "us": ev * 1e3,
                                  "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                                  "kernel": lib.bch_sgemm_kernel_name(m, n, k).decode()}
        del a, b, c
    out["sgemm_shapes"] = shapes
    return out


def _bench_sdpa(dev, T, reps):
    from barracuda_amd import LcgStream, Tensor
    from barracuda_amd import _native as N
    lib, ctx = dev._lib, dev.ctx
    out = {}
    # config 5: SDPA forward B=4, H=32, S=2048, D=128, N(0,1), seed 4, scale 1/sqrt(128)
    Bb, H, S, D = 4, 32, 2048, 128
    s = LcgStream(4, dev)
    q, k, v = (s.normal([Bb, H, S, D]) for _ in range(3))
    o = Tensor.empty([Bb, H, S, D], dev)
    pq, pk, pv, po = (C.c_void_p(t.ptr) for t in (q, k, v, o))
    scale = 1.0 / math.sqrt(D)
    for causal in (0, 1):
        wall, ev = T.run(lambda i: lib.bch_sdpa_fwd(ctx, Bb, H, S, S, D, scale, causal, pq, pk, pv, po),
                         max(5, reps // 2), 2)
        fl = 4.0 * Bb * H * S * S * D if not causal else 4.0 * Bb * H * (S * (S + 1) / 2) * D
        key = "sdpa_causal" if causal else "sdpa_noncausal"
        out[key] = {"ms": ev, "TFLOP/s": fl / (ev * 1e-3) / 1e12,
                    "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                    "traffic": load_traffic(key)}
    del k, v
    # grouped-query attention (ops/grouped_query_attention): the same queries, 8 key/value
    # heads shared by 4 query heads each, through bch_sdpa_fwd_ex (dense [B,H,S,D] layouts)
    Hkv = 8
    kg, vg = s.normal([Bb, Hkv, S, D]), s.normal([Bb, Hkv, S, D])
    lq = N.AttnLayout(H * S * D, S * D, D)
    lkv = N.AttnLayout(Hkv * S * D, S * D, D)
    pkg, pvg = C.c_void_p(kg.ptr), C.c_void_p(vg.ptr)
    wall, ev = T.run(lambda i: lib.bch_sdpa_fwd_ex(ctx, Bb, H, Hkv, S, S, D, scale, 0, pq, lq, pkg, lkv, pvg, lkv,
                                                   po, lq), max(5, reps // 2), 2)
    fl = 4.0 * Bb * H * S * S * D
    out["gqa_hkv8_noncausal"] = {"ms": ev, "TFLOP/s": fl / (ev * 1e-3) / 1e12,
                                 "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS}
    del q, kg, vg, o
    # config 5's shape at wider heads (the reference's attention ops take any head_dim): D = 256 on
    # the fused kernel's widest instance, D = 512 on the chunked GEMM / softmax / GEMM path
    for Dw in (256, 512):
        s = LcgStream(4, dev)
        q, k, v = (s.normal([Bb, H, S, Dw]) for _ in range(3))
        o = Tensor.empty([Bb, H, S, Dw], dev)
        pq, pk, pv, po = (C.c_void_p(t.ptr) for t in (q, k, v, o))
        scale = 1.0 / math.sqrt(Dw)
        for causal in (0, 1):
            wall, ev = T.run(lambda i: lib.bch_sdpa_fwd(ctx, Bb, H, S, S, Dw, scale, causal, pq, pk, pv, po),
                             max(5, reps // 2), 2)
            fl = 4.0 * Bb * H * S * S * Dw if not causal else 4.0 * Bb * H * (S * (S + 1) / 2) * Dw
            key = f"sdpa_d{Dw}_{'causal' if causal else 'noncausal'}"
            out[key] = {"ms": ev, "TFLOP/s": fl / (ev * 1e-3) / 1e12,
                        "mfma_frac": fl / (ev * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                        "path": "fused" if Dw <= 256 else "chunked (GEMM, masked softmax, GEMM)"}
        del q, k, v, o
    return out


def host_cpu() -> dict:
    """What the CPU baselines ran on: the model name from /proc/cpuinfo (what
    lscpu prints as "Model name") and the logical CPU count."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count()}


def _timed(fn, min_s: float = 0.0, min_reps: int = 1):
    """Mean seconds per call of fn() over at least min_reps calls and min_s."""
    reps, t0 = 0, time.perf_counter()
    while reps < min_reps or time.perf_counter() - t0 < min_s:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_baselines(target_s: float = 12.0, extra: bool = True):
    """The reference's CPU paths, restated in oracle/, on this host's cores:
    one entry per BASELINE config (configs 3a/3b/4 on execute_matmul_cpu,
    cpu_executor/executor.rs:241-260, with all cores as rayon uses them;
    softmax_dim and both attention paths serial, as in the reference)."""
    from oracle import bc_oracle as O
    host = host_cpu()
    threads = O.num_threads()
    n = 4096
    rng = O.Lcg(2)
    a, b = rng.uniform((n, n)), rng.uniform((n, n))
    t0 = time.perf_counter()
    O.matmul_cpu_exec_f32(a, b, 0, 16)
    dt = time.perf_counter() - t0
    rows = int(max(16, min(n, 16 * target_s / max(dt, 1e-3))))
    rows = min(n, (rows // threads + 1) * threads)
    t0 = time.perf_counter()
    O.matmul_cpu_exec_f32(a, b, 0, rows)
    dt = time.perf_counter() - t0
    gemm = {"value": 2.0 * rows * n * n / dt / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port", **host,
            "sample": f"rows 0..{rows} of the 4096^3 GEMM (execute_matmul_cpu restated: "
                      f"i-j-p f32 fma, OpenMP over rows as rayon), {dt:.1f} s; rate extrapolates linearly"}
    del a, b
    ex = {}
    if not extra:
        return gemm, ex
    # config 1: the 256^3 matmul on the reference's CPU path, whole
    a2, b2 = O.Lcg(0).uniform((256, 256)), O.Lcg(0).uniform((256, 256))
    O.matmul_cpu_exec_f32(a2, b2, 0, 256)
    dt, reps = _timed(lambda: O.matmul_cpu_exec_f32(a2, b2, 0, 256), 0.5, 5)
    ex["matmul_256"] = {"ms": dt * 1e3, "GFLOP/s": 2.0 * 256 ** 3 / dt / 1e9, "cores": threads, "kind": "port",
                        **host, "sample": f"whole 256^3 matmul (execute_matmul_cpu restated, OpenMP over rows), "
                                          f"mean of {reps} calls; NagaExecutor not run: no Rust toolchain"}
    # config 2: softmax_dim, serial (tensor_axis_ops.rs:67-126 runs on the host thread)
    x = O.Lcg(1).normal((65536, 2048), 0.0, 3.0)
    t0 = time.perf_counter()
    O.softmax_dim_f32(x, 1, 0, 2048)
    dt = time.perf_counter() - t0
    ex["softmax_dim"] = {"GB/s": 2 * 4 * 2048 * 2048 / dt / 1e9, "cores": 1, "kind": "port", **host,
                         "us_full_config_extrapolated": dt * 32 * 1e6,
                         "sample": "rows 0..2048 of 65536x2048 (tensor_axis_ops.rs softmax_dim, serial), "
                                   "x32 extrapolated"}
    del x
    # config 3b: batched 16 x 1024^3, execute_matmul_cpu per batch on a row sample of every batch
    s2 = O.Lcg(2)
    ab, bb = s2.uniform((16, 1024, 1024)), s2.uniform((16, 1024, 1024))
    rb = 4 * threads  # rows per batch in the sample: four per thread
    t0 = time.perf_counter()
    for i in range(16):
        O.matmul_cpu_exec_f32(ab[i], bb[i], 0, rb)
    dt = time.perf_counter() - t0
    fl = 2.0 * 16 * rb * 1024 * 1024
    ex["batched_16x1024"] = {"TFLOP/s": fl / dt / 1e12, "ms_full_config_extrapolated": dt * 1024 / rb * 1e3,
                             "cores": threads, "kind": "port", **host,
                             "sample": f"rows 0..{rb} of each of the 16 batches (execute_matmul_cpu restated, "
                                       f"OpenMP over rows), {dt:.2f} s; x{1024 // rb} extrapolated"}
    del ab, bb
    # config 4: skinny M in {1, 8, 32} x K 4096 x N 11008, whole op (rayon over M rows:
    # at M = 1 only one core has work, as in the reference)
    K, N = 4096, 11008
    for m in (1, 8, 32):
        s3 = O.Lcg(3)
        xs, w = s3.normal((m, K)), s3.normal((K, N), 0.0, 0.02)
        dt, reps = _timed(lambda: O.matmul_cpu_exec_f32(xs, w), 0.3, 2)
        nbytes = 4 * (K * N + m * K + m * N)
        ex[f"skinny_m{m}"] = {"us": dt * 1e6, "GB/s": nbytes / dt / 1e9, "GFLOP/s": 2.0 * m * K * N / dt / 1e9,
                              "cores": min(threads, m), "kind": "port", **host,
                              "sample": f"whole op, mean of {reps} calls (execute_matmul_cpu restated, "
                                        f"OpenMP over the {m} rows)"}
        del xs, w
    # config 5: one (b,h) head of S=2048, D=128 on each attention path, serial, x128
    s4 = O.Lcg(4)
    shape = (1, 1, 2048, 128)
    q, k, v = s4.normal(shape), s4.normal(shape), s4.normal(shape)
    t0 = time.perf_counter()
    O.causal_attention_cpu_f32(q, k, v)
    dt = time.perf_counter() - t0
    ex["causal_attention"] = {"ms_full_config_extrapolated": dt * 1e3 * 128, "cores": 1, "kind": "port", **host,
                              "sample": "1 of 128 heads (causal_attention.rs:52-134, serial), x128 extrapolated"}
    O.set_num_threads(1)
    try:
        t0 = time.perf_counter()
        O.attention_3pass_f32(q, k, v, False)
        dt = time.perf_counter() - t0
    finally:
        O.set_num_threads(threads)
    ex["attention_noncausal"] = {"ms_full_config_extrapolated": dt * 1e3 * 128, "cores": 1, "kind": "port",
                                 **host,
                                 "sample": "1 of 128 heads, the three passes of Attention::execute (K6 scores / "
                                           "sqrt(D), K7 row softmax, K9 P.V; ops/attention/compute.rs:21-111) "
                                           "on the host, serial, x128 extrapolated"}
    return gemm, ex


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="only the headline GEMM")
    ap.add_argument("--skinny-n", type=int, default=11008,
                    help="N of the skinny workload under --only (profiling; the config is 11008)")
    ap.add_argument("--only", default=None,
                    help="comma list of " + ",".join(("gemm",) + WORKLOADS) + ": time just these "
                         "(profiling runs); prints their results as the JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the hot path here is single-GPU (no collectives); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    from barracuda_amd import get_device
    dev = get_device()
    warmer = ClockWarmer(dev)
    if args.only:
        sel = [w.strip() for w in args.only.split(",") if w.strip()]
        res = {}
        if "gemm" in sel:
            g, keep = bench_gemm(dev, args.steps, args.warmup, warmer)
            res["gemm_4096"] = {"TFLOP/s": g["flops"] / (g["kernel_ms"] * 1e-3) / 1e12, "ms": g["kernel_ms"]}
            del keep
        rest = [w for w in sel if w != "gemm"]
        if rest:
            res.update(bench_extra(dev, only=rest, warmer=warmer, skinny_n=args.skinny_n))
        print(json.dumps({"only": sel, "results": res}), flush=True)
        return 0
    log(f"gemm 4096^3: {args.warmup} warmup + {args.steps} timed launches")
    g, keep = bench_gemm(dev, args.steps, args.warmup, warmer)
    value = g["flops"] / (g["wall_ms"] * 1e-3) / 1e12
    achieved = g["flops"] / (g["kernel_ms"] * 1e-3) / 1e12
    log(f"  wall {g['wall_ms']:.3f} ms/step, kernel {g['kernel_ms']:.3f} ms -> {achieved:.1f} TFLOP/s")
    del keep
    extra = None
    if not args.no_extra:
        log("extra configs: softmax, skinny, batched, sdpa, linear, dgemm, norm")
        extra = bench_extra(dev, warmer=warmer)
        for k_, v_ in extra.items():
            log(f"  {k_}: {json.dumps({kk: round(vv, 4) if isinstance(vv, float) else vv for kk, vv in v_.items()})}")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle restatement of the reference CPU path)")
        cpu, cpu_extra = cpu_baselines(extra=not args.no_extra)
        if extra is not None:
            extra["cpu"] = cpu_extra
    rec = {
        "metric": "f32 GEMM TFLOP/s @4096^3 (% FP32 MFMA peak); softmax GB/s; attention fwd ms",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": g["wall_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: U[-1,1) from the reference's rng.rs LCG, seed 2, generated in HBM",
        "config": {"workload": "f32 GEMM C=A.B, M=N=K=4096, row-major (BASELINE configs[2])",
                   "m": 4096, "n": 4096, "k": 4096, "kernel": g["kernel"]},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_MFMA_PEAK_TFLOPS,
                     "traffic": load_traffic("sgemm_4096")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
