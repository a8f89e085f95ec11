"""nn::fused_mlp over the GEMM's fused epilogue (bch_sgemm_ex).

Mirrors crates/barracuda/src/nn/fused_mlp.rs:
  Activation                                     fused_mlp.rs:25-31
  fused_mlp(input, weights, biases, activation)  fused_mlp.rs:38-168
with the same validation order and messages.  The reference records, per
layer, shaders/misc/linear_f64.wgsl (y = x W^T + b) and then
shaders/activation/relu_f64.wgsl over the layer's output, in one submit.
Here each layer is ONE launch: the GEMM adds the bias and applies ReLU in its
epilogue, so the output is written once and never re-read.

Weights may be [out, in] (the linear shader's layout, the product uses them
transposed) or [in, out] (used as they are).  For [in, out] weights that are
not square the reference still indexes the buffer as [out, in]
(linear_f64.wgsl:35 reads weight[out_f * in_features + in_f] whichever branch
of fused_mlp.rs:72-82 matched), which is not x W; this computes x W.
"""
from __future__ import annotations

import ctypes as C
import enum
from typing import Sequence

from . import _native as N
from .error import InvalidInput
from .tensor import Tensor, _check_i32, _same_device

__all__ = ["Activation", "fused_mlp", "linear"]


class Activation(enum.Enum):
    """fused_mlp.rs:25-31: the MLP's activation.  The reference has ReLU
    only; GELU (the tanh form of shaders/activation/gelu_f64.wgsl, the
    activation of transformer MLP blocks) is the same fused epilogue with
    BCH_ACT_GELU."""
    ReLU = "ReLU"
    GELU = "GELU"


def fused_mlp(input: Tensor, weights: Sequence[Tensor], biases: Sequence[Tensor],
              activation: Activation = Activation.ReLU) -> Tensor:
    if len(weights) != len(biases):
        raise InvalidInput(f"fused_mlp: weights len {len(weights)} != biases len {len(biases)}")
    if not weights:
        raise InvalidInput("fused_mlp: at least one layer required")
    shape = input.shape()
    if len(shape) != 2:
        raise InvalidInput(f"fused_mlp: input must be 2D, got {shape}")
    batch, in_features = shape
    layers = []  # (in, out, transb)
    for i, (w, b) in enumerate(zip(weights, biases)):
        ws = w.shape()
        if len(ws) != 2:
            raise InvalidInput(f"fused_mlp: weight[{i}] must be 2D")
        if ws[1] == in_features:
            out_f, in_f, transb = ws[0], ws[1], 1  # [out, in]: x W^T
        elif ws[0] == in_features:
            out_f, in_f, transb = ws[1], ws[0], 0  # [in, out]: x W
        else:
            raise InvalidInput(f"fused_mlp: weight[{i}] shape {ws} incompatible")
        if b.shape() != [out_f]:
            raise InvalidInput(f"fused_mlp: bias[{i}] shape mismatch")
        layers.append((in_f, out_f, transb))
        in_features = out_f
    dev = _same_device(input, *weights, *biases)
    act = {Activation.ReLU: N.BCH_ACT_RELU, Activation.GELU: N.BCH_ACT_GELU}[activation]
    x = input
    for (in_f, out_f, transb), w, b in zip(layers, weights, biases):
        _check_i32("fused_mlp", dev, batch=batch, in_features=in_f, out_features=out_f)
        y = Tensor.empty([batch, out_f], dev)
        if batch * out_f:
            with dev._lock:
                dev.check(dev._lib.bch_sgemm_ex(dev.ctx, transb, batch, out_f, in_f, C.c_void_p(x.ptr),
                                                max(in_f, 1), C.c_void_p(w.ptr),
                                                max(in_f if transb else out_f, 1), C.c_void_p(b.ptr), act,
                                                C.c_void_p(y.ptr), max(out_f, 1)), "fused_mlp")
        x = y
    return x


def linear(input: Tensor, weight: Tensor, bias: Tensor | None = None, activation: Activation | None = None) -> Tensor:
    """One layer of linear_f64.wgsl (y = x W^T + b, W [out, in]) with the
    activation that follows it fused into the GEMM's epilogue: one launch,
    the output written once.  input [batch, in]."""
    shape, ws = input.shape(), weight.shape()
    if len(shape) != 2 or len(ws) != 2 or ws[1] != shape[1]:
        raise InvalidInput(f"linear: input {shape} and weight {ws} (expected [out, {shape[-1] if shape else '?'}])")
    batch, in_f = shape
    out_f = ws[0]
    if bias is not None and bias.shape() != [out_f]:
        raise InvalidInput("linear: bias shape mismatch")
    dev = _same_device(input, weight, *([bias] if bias is not None else []))
    _check_i32("linear", dev, batch=batch, in_features=in_f, out_features=out_f)
    act = {None: N.BCH_ACT_NONE, Activation.ReLU: N.BCH_ACT_RELU, Activation.GELU: N.BCH_ACT_GELU}[activation]
    y = Tensor.empty([batch, out_f], dev)
    if batch * out_f:
        with dev._lock:
            dev.check(dev._lib.bch_sgemm_ex(dev.ctx, 1, batch, out_f, in_f, C.c_void_p(input.ptr), max(in_f, 1),
                                            C.c_void_p(weight.ptr), max(in_f, 1),
                                            C.c_void_p(bias.ptr) if bias is not None else None, act,
                                            C.c_void_p(y.ptr), max(out_f, 1)), "linear")
    return y
