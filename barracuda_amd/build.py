"""Build libbarracuda_hip.so (gfx950) in-tree, plus the code object used by
the dispatch_binary path and the CPU oracle used by the tests.

    python -m barracuda_amd.build          # or __graft_entry__.build()

Outputs (git-ignored, shipped with the tree):
    barracuda_amd/lib/libbarracuda_hip.so
    barracuda_amd/lib/bch_softmax_rows.hsaco
    oracle/libbc_oracle.so                  (test infrastructure only)
    tests/cpp/bch_host_tests                (C++ host-API tests)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"
ARCH = os.environ.get("BARRACUDA_HIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# Packed-FP32 VALU ops are disabled for all device code: some of their forms
# have given wrong results on this hardware, with no error.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
SOURCES = ["bch_runtime.hip", "softmax_rows.hip", "sgemm_mfma.hip",
           "sgemm_skinny.hip", "sdpa_fwd.hip", "sdpa_wide.hip", "dgemm_mfma.hip",
           "rng_fill.hip", "copy.hip", "elementwise.hip", "layer_norm.hip", "head_permute.hip",
           "softmax_f64.hip"]
# Per-file code-generation flags.  The skinny GEMM keeps its MFMA
# accumulators in VGPRs: with the default heuristics the compiler parks them
# in AGPRs and copies them back and forth inside the k loop (measured: 716
# v_accvgpr moves per loop, M=32 48.3 -> 43.4 us).  The big GEMM needs all
# 256 AGPRs for its 256x256 tile, so the flag is not global.
FILE_FLAGS = {
    "sgemm_skinny.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip(verbose: bool = True) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = []
    for src in SOURCES:
        obj = OBJ / (Path(src).stem + ".o")
        jobs.append([HIPCC, *DEVICE_FLAGS, *FILE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)])
    # the code object for bch_launch_code_object (dispatch_binary)
    hsaco = LIB / "bch_softmax_rows.hsaco"
    jobs.append([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "--genco",
                 "--no-gpu-bundle-output",
                 "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                 str(CSRC / "softmax_rows.hip"), "-o", str(hsaco)])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()
    so = LIB / "libbarracuda_hip.so"
    tmp = LIB / "libbarracuda_hip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *[str(OBJ / (Path(s).stem + ".o")) for s in SOURCES],
          "-Wl,-rpath,/opt/rocm/lib", "-ldl"])
    os.replace(tmp, so)
    if verbose:
        print(f"built {so.relative_to(ROOT)} and {hsaco.relative_to(ROOT)} for {ARCH}")
    return so


def build_host_tests(verbose: bool = True) -> Path:
    """The C++ host-API tests (tests/cpp/test_ops.cpp) against include/barracuda_hip_ops.hpp."""
    exe = ROOT / "tests" / "cpp" / "bch_host_tests"
    _run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", f"-I{ROOT / 'include'}",
          str(ROOT / "tests" / "cpp" / "test_ops.cpp"), f"-L{LIB}", "-lbarracuda_hip",
          "-Wl,-rpath,$ORIGIN/../../barracuda_amd/lib", "-o", str(exe)])
    if verbose:
        print(f"built {exe.relative_to(ROOT)}")
    return exe


def build_oracle(verbose: bool = True) -> Path:
    odir = ROOT / "oracle"
    _run(["make", "-s", "-B", "-C", str(odir)])
    so = odir / "libbc_oracle.so"
    if verbose:
        print(f"built {so.relative_to(ROOT)}")
    return so


SAN = LIB / "sanitize"
# Host-code sanitizers for the C ABI's runtime: every flag applies to the
# host pass only (each -fsanitize= right after -Xarch_host); device code is
# built exactly as in build_hip.
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
CLANGXX = "/opt/rocm/llvm/bin/clang++"


def build_sanitized(verbose: bool = True) -> Path:
    """AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code,
    run on the CPU by tests/test_sanitizers.py:
      oracle/_asan/libbc_oracle.so              (gcc; `make -C oracle asan`)
      barracuda_amd/lib/sanitize/libbarracuda_hip.so   (bch_runtime.hip's host
          pass sanitized, linked against the clang ASan runtime; the kernels'
          objects are build_hip's)
      barracuda_amd/lib/sanitize/bch_host_tests (tests/cpp/test_ops.cpp,
          clang++, same runtime)
    Needs build_hip's objects."""
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"])
    SAN.mkdir(parents=True, exist_ok=True)
    rt = SAN / "bch_runtime.o"
    _run([HIPCC, f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", "-fPIC",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *HOST_SAN,
          "-c", str(CSRC / "bch_runtime.hip"), "-o", str(rt)])
    objs = [str(OBJ / (Path(s).stem + ".o")) for s in SOURCES if s != "bch_runtime.hip"]
    so = SAN / "libbarracuda_hip.so"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libasan", *HOST_SAN[:4],
          "-o", str(so), str(rt), *objs, "-Wl,-rpath,/opt/rocm/lib", "-ldl"])
    asan_rt = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                             text=True).stdout.strip()
    exe = SAN / "bch_host_tests"
    _run([CLANGXX, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
          "-fno-sanitize-recover=undefined", "-shared-libasan", f"-I{ROOT / 'include'}",
          str(ROOT / "tests" / "cpp" / "test_ops.cpp"), f"-L{SAN}", "-lbarracuda_hip",
          f"-Wl,-rpath,{SAN}", f"-Wl,-rpath,{Path(asan_rt).parent}", "-o", str(exe)])
    if verbose:
        print(f"built sanitized host builds under {SAN.relative_to(ROOT)} and oracle/_asan")
    return SAN


def build_all(verbose: bool = True) -> None:
    build_oracle(verbose)
    build_hip(verbose)
    build_host_tests(verbose)
    build_sanitized(verbose)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
