"""The C++ host API (include/barracuda_hip_ops.hpp) tested the way the
reference tests its Rust ops: tests/cpp/test_ops.cpp, built by
barracuda_amd.build into tests/cpp/bch_host_tests."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "cpp" / "bch_host_tests"


def _run(mode: str) -> str:
    assert EXE.exists(), f"{EXE} not built: python -m barracuda_amd.build"
    r = subprocess.run([str(EXE), mode], capture_output=True, text=True, timeout=240)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    return r.stdout


def test_cpp_host_validation_without_device():
    out = _run("--cpu")
    assert "PASS validate_matmul_inner_dim_mismatch" in out
    assert "PASS validate_fused_mlp" in out
    assert "PASS validate_layer_norm" in out
    assert "PASS no_device_is_an_error_value" in out


@pytest.mark.gpu
def test_cpp_host_ops_on_gpu():
    out = _run("--gpu")
    for name in ("test_matmul_basic", "test_batch_matmul_basic", "test_softmax_vs_cpu",
                 "test_softmax_dim_rows_and_columns", "test_attention_basic", "test_sdpa_and_causal",
                 "test_fault_injection_shape_mismatch", "test_grouped_query_attention_basic",
                 "test_mha_basic_and_cross_attention", "test_fused_mlp_two_layers",
                 "test_gemm_f64_basic_transpose_batched",
                 "test_relu_gelu_layer_norm", "test_fused_mlp_gelu", "test_session_head_split_concat"):
        assert f"PASS {name}" in out
