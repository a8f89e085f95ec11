"""barracuda_amd -- MI355X (gfx950) implementation of barraCuda's dense ML-ops
hot path: f32 matmul / batched matmul, row softmax, fused attention forward.

The compute lives in libbarracuda_hip.so (C ABI: include/barracuda_hip.h);
this package is the host side that mirrors the reference's op API.
"""
from .error import (BarracudaError, CastOverflow, DeviceError, DeviceLost, DeviceNotAvailable,
                    ExecutionError, InvalidInput, InvalidOperation, InvalidShape, OutOfMemory,
                    ShapeMismatch, UnsupportedOperation)
from . import ipc, linalg, nn
from .linalg import F64Buffer, GemmCachedF64, GemmF64
from .nn import Activation, fused_mlp
from .session import AttentionDims, SessionTensor, TensorSession
from .tensor import (GELU, Attention, BatchMatMul, CausalAttention, FlashAttention, GroupedQueryAttention,
                     HipDevice, LayerNorm, LcgStream, MatMul, MatmulTiled, MultiHeadAttention, ReLU,
                     ScaledDotProductAttention, Softmax, Tensor, get_device)

__all__ = [
    "BarracudaError", "CastOverflow", "DeviceError", "DeviceLost", "DeviceNotAvailable",
    "ExecutionError", "InvalidInput", "InvalidOperation", "InvalidShape", "OutOfMemory",
    "ShapeMismatch", "UnsupportedOperation", "AttentionDims", "SessionTensor", "TensorSession",
    "Activation", "fused_mlp", "nn", "linalg", "ipc", "F64Buffer", "GemmCachedF64", "GemmF64",
    "Attention", "BatchMatMul", "CausalAttention", "FlashAttention", "GroupedQueryAttention", "HipDevice",
    "MatMul", "MultiHeadAttention",
    "MatmulTiled", "ScaledDotProductAttention", "Softmax", "Tensor", "get_device", "LcgStream",
    "ReLU", "GELU", "LayerNorm",
]
