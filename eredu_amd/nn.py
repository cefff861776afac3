"""Linear-layer dispatch: which layer a projection gets for its stored encoding.

Mirrors ``eredu/src/backend/mlx/nn/linear.rs:47-105``
(``unloaded_maybe_quantized_linear[_with_dtype]``) and ``MlxBackend::linear``
(``eredu/src/backend/mlx/nn/shared.rs:178-195``): a ``LinearSpec`` whose
``quantization`` is

* ``None``                          -> a dense ``Linear`` (weight [out, in]),
* ``WeightQuantization.GgufIQuant`` -> ``QuantizedLinear.unloaded_iq`` (native
  GGML block rows, executed by the native GGUF linear),
* affine or MXFP4                   -> ``QuantizedLinear.unloaded_with_mode``.

Layers are created unloaded (placeholders of the right shapes) and filled
from a checkpoint with ``load_parameters``; ``forward`` then dispatches to the
matching device kernel (``QuantizedLinear.forward``).  The dense ``Linear`` is
the non-quantized branch a model may also hold (embeddings-sized heads, tied
weights); its product is a plain device matmul and is not part of this
library's quantized path.
"""
from __future__ import annotations

import dataclasses
from typing import Optional, Union

import torch

from ._native import EreduError
from .checkpoint import WeightQuantization
from .quantization import QuantizationMode, QuantizedLinear


@dataclasses.dataclass(frozen=True)
class LinearSpec:
    """eredu-nn/src/lib.rs:64-77: shape and checkpoint identity of a projection."""

    input: int
    output: int
    bias: bool = False
    weight_name: str = ""
    quantization: Optional[WeightQuantization] = None


class Linear:
    """Dense linear layer (safemlx/src/nn/linear.rs): y = x . W^T + b."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        self.weight = weight
        self.bias = bias

    @classmethod
    def unloaded(cls, input_dims: int, output_dims: int, bias: bool, dtype: torch.dtype = torch.float32,
                 device=None) -> "Linear":
        """Placeholder of the checkpoint's shapes (linear.rs:75-91)."""
        dev = torch.device("cuda") if device is None else device
        w = torch.zeros((output_dims, input_dims), dtype=dtype, device=dev)
        b = torch.zeros((output_dims,), dtype=dtype, device=dev) if bias else None
        return cls(w, b)

    def shape(self):
        return tuple(self.weight.shape)

    def load_parameters(self, params: dict) -> None:
        for name in ("weight", "bias"):
            if name not in params:
                continue
            cur, new = getattr(self, name), params[name]
            if cur is None:
                raise EreduError(f"layer has no parameter {name!r}")
            if tuple(new.shape) != tuple(cur.shape):
                raise EreduError(f"parameter {name!r}: shape {tuple(new.shape)}, expected {tuple(cur.shape)}")
            setattr(self, name, new)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = x @ self.weight.to(x.dtype).t()
        if self.bias is not None:
            y = y + self.bias
        return y

    __call__ = forward


MaybeQuantizedLinear = Union[Linear, QuantizedLinear]


def mlx_quantization_mode(config: WeightQuantization) -> QuantizationMode:
    """eredu/src/backend/mlx/runtime/checkpoint/quantization.rs:226-234."""
    if config.mode == "affine":
        return QuantizationMode.Affine
    if config.mode == "mxfp4":
        return QuantizationMode.MxFp4
    raise EreduError("checkpoint-native GGML blocks cannot be produced by dense quantization")


def unloaded_maybe_quantized_linear_with_dtype(input_dims: int, output_dims: int, bias: bool,
                                               quantization: Optional[WeightQuantization],
                                               dense_dtype: torch.dtype = torch.float32,
                                               device=None) -> MaybeQuantizedLinear:
    """eredu/src/backend/mlx/nn/linear.rs:64-101."""
    if quantization is not None:
        quantization.validate()
        iq = quantization.gguf_iquant()
        if iq is not None:
            return QuantizedLinear.unloaded_iq(input_dims, output_dims, iq[0], iq[1], bias, device)
        return QuantizedLinear.unloaded_with_mode(input_dims, output_dims, quantization.group_size,
                                                  quantization.bits, mlx_quantization_mode(quantization), bias,
                                                  device)
    return Linear.unloaded(input_dims, output_dims, bias, dense_dtype, device)


def unloaded_maybe_quantized_linear(input_dims: int, output_dims: int, bias: bool,
                                    quantization: Optional[WeightQuantization], device=None) -> MaybeQuantizedLinear:
    """eredu/src/backend/mlx/nn/linear.rs:47-62 (dense placeholders in f32)."""
    return unloaded_maybe_quantized_linear_with_dtype(input_dims, output_dims, bias, quantization, torch.float32,
                                                      device)


def linear(spec: LinearSpec, device=None) -> MaybeQuantizedLinear:
    """MlxBackend::linear (eredu/src/backend/mlx/nn/shared.rs:186-195)."""
    return unloaded_maybe_quantized_linear(spec.input, spec.output, spec.bias, spec.quantization, device)
