"""Shared test setup.

Markers: `gpu` tests need an MI355X and call through the C ABI
(libbarracuda_hip.so); everything else runs on the CPU.
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "reference_vectors.json"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP kernels")


@pytest.fixture(scope="session")
def golden():
    return json.loads(GOLDEN.read_text())


def f32(x: float) -> float:
    return struct.unpack("f", struct.pack("f", x))[0]


def ramp(n: int, spec) -> np.ndarray:
    """f32(i * f32(scale) + offset) for i < n (the reference tests' ramps)."""
    scale, off = spec
    i = np.arange(n, dtype=np.float64)
    return (i * np.float64(np.float32(scale)) + off).astype(np.float32)


def case_inputs(case):
    """(a, b) float32 arrays of a golden matmul case."""
    ash, bsh = case["a_shape"], case["b_shape"]
    if "a_ramp" in case:
        a = ramp(int(np.prod(ash)), case["a_ramp"]).reshape(ash)
        b = ramp(int(np.prod(bsh)), case["b_ramp"]).reshape(bsh)
    else:
        a = np.array(case["a"], dtype=np.float32).reshape(ash)
        b = np.array(case["b"], dtype=np.float32).reshape(bsh)
    return a, b


@pytest.fixture(scope="session")
def dev():
    """The default HIP device; GPU tests fail loudly if it is missing."""
    from barracuda_amd import get_device
    return get_device()
