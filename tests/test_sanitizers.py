"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the
CPU (barracuda_amd.build.build_sanitized makes the builds):

  * the oracle (oracle/_asan/libbc_oracle.so, gcc) runs the oracle test
    files in a child process with gcc's ASan/UBSan runtimes preloaded;
  * the C ABI's host code (bch_runtime.hip's host pass, clang) runs the C-ABI
    validation tests (ctypes) with clang's ASan runtime preloaded;
  * the C++ host API (tests/cpp/test_ops.cpp over that runtime) runs in its
    --cpu mode.

Leak detection is off: the HIP runtime keeps process-lifetime allocations.
Device code is not sanitized (GPU sanitizers are not available here)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SAN = ROOT / "barracuda_amd" / "lib" / "sanitize"
ORACLE_ASAN = ROOT / "oracle" / "_asan" / "libbc_oracle.so"


def _tool_file(cmd: list[str]) -> str:
    try:
        out = subprocess.run(cmd, capture_output=True, text=True, timeout=30).stdout.strip()
    except (OSError, subprocess.TimeoutExpired):
        return ""
    return out if out and os.path.isabs(out) and os.path.exists(out) else ""


def _env(preload: list[str], **extra) -> dict:
    env = dict(os.environ)
    env["LD_PRELOAD"] = ":".join(preload)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.update(extra)
    return env


def _need(path: Path):
    if not path.exists():
        pytest.skip(f"{path} not built: python -m barracuda_amd.build")


def _check(r: subprocess.CompletedProcess):
    out = r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in out, out[-4000:]
    assert "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]


def test_oracle_under_asan_ubsan():
    _need(ORACLE_ASAN)
    asan = _tool_file(["gcc", "-print-file-name=libasan.so"])
    ubsan = _tool_file(["gcc", "-print-file-name=libubsan.so"])
    if not asan or not ubsan:
        pytest.skip("gcc's ASan/UBSan runtimes are not installed")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "tests/test_oracle.py", "tests/test_oracle_callers.py"],
                       cwd=ROOT, env=_env([asan, ubsan], BC_ORACLE_LIB=str(ORACLE_ASAN)),
                       capture_output=True, text=True, timeout=600)
    _check(r)
    assert " passed" in r.stdout


def test_c_abi_host_code_under_asan_ubsan():
    _need(SAN / "libbarracuda_hip.so")
    asan = _tool_file(["/opt/rocm/llvm/bin/clang++", "-print-file-name=libclang_rt.asan-x86_64.so"])
    if not asan:
        pytest.skip("clang's ASan runtime is not installed")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                        "tests/test_capi.py", "tests/test_session_host.py"],
                       cwd=ROOT, env=_env([asan], BARRACUDA_HIP_LIB=str(SAN / "libbarracuda_hip.so")),
                       capture_output=True, text=True, timeout=600)
    _check(r)
    assert " passed" in r.stdout


def test_cpp_host_api_under_asan_ubsan():
    exe = SAN / "bch_host_tests"
    _need(exe)
    r = subprocess.run([str(exe), "--cpu"], env=_env([]), capture_output=True, text=True, timeout=240)
    _check(r)
    assert "PASS no_device_is_an_error_value" in r.stdout and " 0 failed" in r.stdout
