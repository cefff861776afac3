"""Host-side mirror of eredu-gguf's tensor conversion on the gfx950 kernels.

Follows ``eredu-gguf/src/convert.rs`` (``convert_affine``, ``AffineTensor``)
and ``eredu-gguf/src/format.rs`` (``GgmlType``, ``TensorDescriptor``,
``Endian``) for the block types the device path covers: Q4_0, Q8_0 and Q4_K.
The raw block payload is a uint8 tensor on the GPU (what a loader copies to
the device); outputs are GPU tensors.  Conversion and dequantization run in
the HIP library; there is no host path.
"""
from __future__ import annotations

import dataclasses
import enum
from typing import List, Optional

import torch

from . import _native
from ._native import EreduError, check


class GgmlType(enum.IntEnum):
    """Codes of eredu-gguf/src/format.rs:297-330 handled on the device."""

    Q4_0 = 2
    Q8_0 = 8
    Q4K = 12

    def block_and_bytes(self):
        """(values per block, bytes per block), format.rs:368-400."""
        return {GgmlType.Q4_0: (32, 18), GgmlType.Q8_0: (32, 34), GgmlType.Q4K: (256, 144)}[self]

    def has_native_execution(self) -> bool:
        """format.rs:423-428: Q4_K and Q8_0 stay native in eredu; Q4_0 does not."""
        return self in (GgmlType.Q4K, GgmlType.Q8_0)


def affine_config(ty: GgmlType):
    """(bits, group_size) of the affine form, convert.rs:142-152."""
    return {GgmlType.Q4_0: (4, 32), GgmlType.Q8_0: (8, 32), GgmlType.Q4K: (4, 32)}[ty]


class Endian(enum.IntEnum):
    Little = _native.EQ_ENDIAN_LITTLE
    Big = _native.EQ_ENDIAN_BIG


class DequantDefinition(enum.IntEnum):
    """AFFINE: convert_affine + AffineTensor::dequantize (convert.rs:43-56,81-101);
    NATIVE: the native decoders (safemlx/src/native_quantization.rs:3445-3469,3539-3542)."""

    Affine = _native.EQ_DEQUANT_AFFINE
    Native = _native.EQ_DEQUANT_NATIVE


@dataclasses.dataclass
class TensorDescriptor:
    """format.rs:431-453; ``dimensions`` in GGML order (fastest first)."""

    name: str
    dimensions: List[int]
    ggml_type: GgmlType
    byte_len: int

    def mlx_shape(self) -> List[int]:
        return list(reversed(self.dimensions))


@dataclasses.dataclass
class AffineTensor:
    """convert.rs:59-70: packed u32 weights and f16 scale/bias bit patterns
    (as torch.float16 tensors on the GPU)."""

    weight_shape: List[int]
    scale_shape: List[int]
    bits: int
    group_size: int
    weights: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """f32(scale) * code + f32(bias) (convert.rs:81-101), written as ``dtype``."""
        from .quantization import dequantize_with_mode

        rows = self.weights.shape[0]
        return dequantize_with_mode(
            self.weights.view(rows, -1), self.scales.view(rows, -1), self.biases.view(rows, -1),
            self.group_size, self.bits, dtype=dtype,
        ).view(*self.weight_shape[:-1], -1)


def _rows_cols(desc: TensorDescriptor):
    shape = desc.mlx_shape()
    if not shape:
        raise EreduError(f"tensor '{desc.name}': quantized scalar is invalid")
    cols = shape[-1]
    rows = 1
    for d in shape[:-1]:
        rows *= d
    return shape, rows, cols


def _check_raw(desc: TensorDescriptor, raw: torch.Tensor) -> None:
    if raw.dtype != torch.uint8 or not raw.is_cuda:
        raise EreduError("raw GGUF payload must be a uint8 tensor on the GPU")
    if raw.numel() != desc.byte_len:
        raise EreduError(f"tensor '{desc.name}': payload length does not match descriptor")


def convert_affine(desc: TensorDescriptor, raw: torch.Tensor, endian: Endian = Endian.Little) -> AffineTensor:
    """GGML blocks -> MLX affine triple, byte-identical to
    eredu_gguf::convert_affine (convert.rs:318-465); C ABI eq_gguf_convert_affine."""
    ty = GgmlType(desc.ggml_type)
    _check_raw(desc, raw)
    shape, rows, cols = _rows_cols(desc)
    bits, gs = affine_config(ty)
    if cols % gs != 0:
        raise EreduError(f"tensor '{desc.name}': last dimension is not divisible by group size {gs}")
    raw = raw.contiguous()
    dev = raw.device
    weights = torch.empty((rows, cols * bits // 32), dtype=torch.int32, device=dev)
    scales = torch.empty((rows, cols // gs), dtype=torch.float16, device=dev)
    biases = torch.empty_like(scales)
    check(
        _native.lib().eq_gguf_convert_affine(
            weights.data_ptr(), scales.data_ptr(), biases.data_ptr(), raw.data_ptr(), raw.numel(),
            int(ty), rows, cols, int(endian), torch.cuda.current_stream().cuda_stream,
        )
    )
    weight_shape = shape[:-1] + [cols * bits // 32]
    scale_shape = shape[:-1] + [cols // gs]
    return AffineTensor(weight_shape, scale_shape, bits, gs, weights.view(*weight_shape),
                        scales.view(*scale_shape), biases.view(*scale_shape))


def dequantize(
    desc: TensorDescriptor,
    raw: torch.Tensor,
    endian: Endian = Endian.Little,
    definition: DequantDefinition = DequantDefinition.Affine,
    dtype: torch.dtype = torch.bfloat16,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Dense dequant of GGML blocks (bf16 = round-to-nearest-even image of the
    reference's f32 values); C ABI eq_gguf_dequantize."""
    ty = GgmlType(desc.ggml_type)
    _check_raw(desc, raw)
    shape, rows, cols = _rows_cols(desc)
    if dtype not in (torch.bfloat16, torch.float32):
        raise EreduError("dense output dtype must be bfloat16 or float32")
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=raw.device)
    elif out.dtype != dtype or list(out.shape) != shape or not out.is_contiguous():
        raise EreduError("out has the wrong dtype, shape or layout")
    code = _native.EQ_DTYPE_BF16 if dtype == torch.bfloat16 else _native.EQ_DTYPE_F32
    check(
        _native.lib().eq_gguf_dequantize(
            out.data_ptr(), raw.contiguous().data_ptr(), raw.numel(), int(ty), rows, cols, int(endian),
            int(definition), code, torch.cuda.current_stream().cuda_stream,
        )
    )
    return out


def linear(x: torch.Tensor, desc: TensorDescriptor, raw: torch.Tensor, endian: Endian = Endian.Little) -> torch.Tensor:
    """y = x . W^T with W the GGUF tensor of ``desc`` decoded by the native
    definition, straight from its Q4_K or Q8_0 blocks (no affine expansion):
    NativeQuantizedTensor::linear with transpose = true
    (safemlx/src/native_quantization.rs:741-772); C ABI eq_gguf_linear.
    x is bf16 [..., K] on the GPU; W's MLX shape is [N, K]."""
    ty = GgmlType(desc.ggml_type)
    _check_raw(desc, raw)
    shape, N, K = _rows_cols(desc)
    if len(shape) != 2:
        raise EreduError(f"tensor '{desc.name}': native linear expects a single logical matrix")
    if x.dtype != torch.bfloat16 or not x.is_cuda or x.shape[-1] != K:
        raise EreduError(f"native linear expected a bf16 CUDA input with trailing dimension {K}")
    x2 = x.reshape(-1, K).contiguous()
    y = torch.empty((x2.shape[0], N), dtype=torch.bfloat16, device=x.device)
    check(
        _native.lib().eq_gguf_linear(
            y.data_ptr(), x2.data_ptr(), raw.contiguous().data_ptr(), raw.numel(), int(ty), x2.shape[0], N, K,
            int(endian), _native.EQ_DTYPE_BF16, torch.cuda.current_stream().cuda_stream,
        )
    )
    return y.reshape(*x.shape[:-1], N)
