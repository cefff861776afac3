"""Host-side mirror of eredu-gguf's tensor conversion on the gfx950 kernels.

Follows ``eredu-gguf/src/convert.rs`` (``convert_affine``, ``AffineTensor``)
and ``eredu-gguf/src/format.rs`` (``GgmlType``, ``TensorDescriptor``,
``Endian``) for the block types the device path covers: Q4_0, Q4_1, Q5_0,
Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K (every type with an affine form).
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
    """GGML tensor type codes (eredu-gguf/src/format.rs:295-365).  The device
    path converts and dequantizes every type with an affine form, dequantizes
    IQ4_NL / IQ4_XS, and executes Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and
    IQ4_XS blocks natively; the rest are named so that routing
    (``conversion_kind``) covers every code the container holds."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    IQ2XXS = 16
    IQ2XS = 17
    IQ3XXS = 18
    IQ1S = 19
    IQ4NL = 20
    IQ3S = 21
    IQ2S = 22
    IQ4XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1M = 29
    BF16 = 30
    MXFP4 = 39

    def block_and_bytes(self):
        """(values per block, bytes per block), format.rs:366-400."""
        return _BLOCK_AND_BYTES[self]

    def is_iq(self) -> bool:
        """The nine on-disk IQ encodings (format.rs:403-416)."""
        return self in _IQ_TYPES

    def has_native_execution(self) -> bool:
        """format.rs:423-428: encodings that stay in their blocks when converted
        (Q4_K, Q5_K, Q6_K, Q5_1, Q8_0 and the IQ types)."""
        return self in (GgmlType.Q4K, GgmlType.Q5K, GgmlType.Q6K, GgmlType.Q5_1, GgmlType.Q8_0) or self.is_iq()

    def has_device_kernels(self) -> bool:
        """Encodings this library dequantizes (and, with an affine form,
        convert.rs:142-152, converts): the ten affine types, IQ4_NL, IQ4_XS."""
        return affine_config(self) is not None or self in (GgmlType.IQ4NL, GgmlType.IQ4XS)

    def has_device_linear(self) -> bool:
        """Encodings this library multiplies straight from their blocks
        (eq_gguf_linear): the non-IQ encodings eredu executes natively."""
        return self in (GgmlType.Q8_0, GgmlType.Q4K, GgmlType.Q5K, GgmlType.Q6K, GgmlType.Q5_1, GgmlType.IQ4NL,
                        GgmlType.IQ4XS)


_BLOCK_AND_BYTES = {
    GgmlType.F32: (1, 4), GgmlType.F16: (1, 2), GgmlType.BF16: (1, 2), GgmlType.I16: (1, 2), GgmlType.I8: (1, 1),
    GgmlType.I32: (1, 4), GgmlType.I64: (1, 8), GgmlType.F64: (1, 8),
    GgmlType.Q4_0: (32, 18), GgmlType.Q4_1: (32, 20), GgmlType.Q5_0: (32, 22), GgmlType.Q5_1: (32, 24),
    GgmlType.Q8_0: (32, 34), GgmlType.Q2K: (256, 84), GgmlType.Q3K: (256, 110), GgmlType.Q4K: (256, 144),
    GgmlType.Q5K: (256, 176), GgmlType.Q6K: (256, 210), GgmlType.IQ2XXS: (256, 66), GgmlType.IQ2XS: (256, 74),
    GgmlType.IQ3XXS: (256, 98), GgmlType.IQ1S: (256, 50), GgmlType.IQ4NL: (32, 18), GgmlType.IQ3S: (256, 110),
    GgmlType.IQ2S: (256, 82), GgmlType.IQ4XS: (256, 136), GgmlType.IQ1M: (256, 56), GgmlType.MXFP4: (32, 17),
}
_IQ_TYPES = (GgmlType.IQ2XXS, GgmlType.IQ2XS, GgmlType.IQ3XXS, GgmlType.IQ1S, GgmlType.IQ4NL, GgmlType.IQ3S,
             GgmlType.IQ2S, GgmlType.IQ4XS, GgmlType.IQ1M)
_DENSE_DTYPES = {GgmlType.F32: torch.float32, GgmlType.F16: torch.float16, GgmlType.BF16: torch.bfloat16,
                 GgmlType.I8: torch.int8, GgmlType.I16: torch.int16, GgmlType.I32: torch.int32,
                 GgmlType.I64: torch.int64, GgmlType.F64: torch.float64}


def ggml_type_from_code(code: int) -> GgmlType:
    """GgmlType::from_code; a code outside the table is UnsupportedTensorType."""
    try:
        return GgmlType(code)
    except ValueError:
        raise EreduError(f"unsupported GGML tensor type {code}") from None


def affine_config(ty: GgmlType):
    """(bits, group_size) of the affine form (convert.rs:142-152), or None."""
    return {GgmlType.Q2K: (2, 16), GgmlType.Q3K: (3, 16), GgmlType.Q4_0: (4, 32), GgmlType.Q4_1: (4, 32),
            GgmlType.Q4K: (4, 32), GgmlType.Q5_0: (5, 32), GgmlType.Q5_1: (5, 32), GgmlType.Q5K: (5, 32),
            GgmlType.Q6K: (6, 16), GgmlType.Q8_0: (8, 32)}.get(GgmlType(ty))


@dataclasses.dataclass(frozen=True)
class ConversionKind:
    """How eredu-gguf converts a tensor (convert.rs:104-140): ``kind`` is
    "dense" (with ``dtype``), "native" (kept in its GGML blocks, the
    reference's ConversionKind::IQuant), "mxfp4", or "affine" (with ``bits``
    and ``group_size``)."""

    kind: str
    dtype: Optional[torch.dtype] = None
    bits: int = 0
    group_size: int = 0


def conversion_kind(ty: GgmlType, endian: "Endian") -> ConversionKind:
    """Routing of convert.rs:125-140: dense types stay dense; IQ types and,
    in little-endian files, the natively executable encodings (Q4_K, Q8_0,
    ...) stay in their blocks; MXFP4 has its own form; everything else with
    an affine geometry is expanded to the affine triple."""
    ty = GgmlType(ty)
    if ty in _DENSE_DTYPES:
        return ConversionKind("dense", dtype=_DENSE_DTYPES[ty])
    if ty.is_iq() or (Endian(endian) == Endian.Little and ty.has_native_execution()):
        return ConversionKind("native")
    if ty == GgmlType.MXFP4:
        return ConversionKind("mxfp4")
    cfg = affine_config(ty)
    if cfg is None:
        raise EreduError(f"unsupported GGML tensor type {int(ty)}")
    return ConversionKind("affine", bits=cfg[0], group_size=cfg[1])


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


def _device_type(desc: TensorDescriptor) -> GgmlType:
    ty = ggml_type_from_code(int(desc.ggml_type))
    if not ty.has_device_kernels():
        raise EreduError(f"tensor '{desc.name}': GGML type {int(ty)} has no device kernels "
                         f"(types with an affine form only)")
    return ty


def _check_raw(desc: TensorDescriptor, raw: torch.Tensor) -> None:
    if raw.dtype != torch.uint8 or not raw.is_cuda:
        raise EreduError("raw GGUF payload must be a uint8 tensor on the GPU")
    if raw.numel() != desc.byte_len:
        raise EreduError(f"tensor '{desc.name}': payload length does not match descriptor")


def convert_affine(desc: TensorDescriptor, raw: torch.Tensor, endian: Endian = Endian.Little) -> AffineTensor:
    """GGML blocks -> MLX affine triple, byte-identical to
    eredu_gguf::convert_affine (convert.rs:318-564); C ABI eq_gguf_convert_affine."""
    ty = _device_type(desc)
    if affine_config(ty) is None:  # convert.rs:329-330
        raise EreduError(f"tensor '{desc.name}': tensor encoding has no affine conversion")
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
    ty = _device_type(desc)
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


def embedding(
    indices: torch.Tensor,
    desc: TensorDescriptor,
    raw: torch.Tensor,
    endian: Endian = Endian.Little,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Rows ``indices`` of the GGUF tensor of ``desc`` decoded by the native
    definition, shape indices.shape + [cols], float32 like the reference (or
    bfloat16, its round-to-nearest-even image): NativeQuantizedTensor::embedding
    (safemlx/src/native_quantization.rs:774-789, 915-939); C ABI
    eq_gguf_embedding.  An index outside [0, rows) raises the reference's
    error (checked here, one device read of the ids, as the reference
    evaluates them on the host)."""
    ty = _device_type(desc)
    _check_raw(desc, raw)
    _, rows, cols = _rows_cols(desc)
    if dtype not in (torch.bfloat16, torch.float32):
        raise EreduError("embedding output dtype must be bfloat16 or float32")
    ids = indices.to(device=raw.device, dtype=torch.int32).contiguous()
    flat = ids.view(-1)
    bad = ((flat < 0) | (flat >= rows)).nonzero()
    if bad.numel():
        raise EreduError(f"native embedding index {int(flat[int(bad[0])].item())} is outside 0..{rows}")
    out = torch.empty(list(ids.shape) + [cols], dtype=dtype, device=raw.device)
    code = _native.EQ_DTYPE_BF16 if dtype == torch.bfloat16 else _native.EQ_DTYPE_F32
    check(
        _native.lib().eq_gguf_embedding(
            out.data_ptr(), raw.contiguous().data_ptr(), raw.numel(), int(ty), rows, cols, ids.data_ptr(),
            ids.numel(), int(endian), code, torch.cuda.current_stream().cuda_stream,
        )
    )
    return out


def native_grouped_linear(input: torch.Tensor, weight: "NativeTensor", group_ids: torch.Tensor) -> torch.Tensor:
    """y[r] = input[r] . W[group_ids[r]]^T for an expert bank W [experts, N, K]
    kept in its GGUF blocks: safemlx's native_grouped_linear
    (safemlx/src/native_quantization.rs:1039-1072; its CPU loop :1002-1037),
    as eredu's MoE calls it on the routes' sorted expert ids
    (eredu/src/backend/mlx/nn/moe.rs:1080-1092).  bf16 input [routes, K] ->
    bf16 [routes, N]; C ABI eq_gguf_grouped_linear.  The reference's shape
    and expert-range errors are raised here (one device read of the ids, as
    the reference evaluates them on the host); whether they are sorted is
    read the same way and picks the grouped matrix-core path."""
    shape = list(weight.shape)
    if input.dim() != 2 or group_ids.dim() != 1 or input.shape[0] != group_ids.shape[0] or len(shape) != 3 or \
            input.shape[1] != shape[2]:
        raise EreduError(f"native grouped linear shape mismatch: input {list(input.shape)}, ids "
                         f"{list(group_ids.shape)}, weight {shape}")
    experts, N, K = shape
    if input.dtype != torch.bfloat16:
        raise EreduError("native GGUF grouped linear takes bfloat16 activations")
    if not input.is_cuda or input.device != weight.data.device:
        raise EreduError("native GGUF grouped linear expected a CUDA input on the weight's device")
    ty = _device_type(weight.descriptor())
    _check_raw(weight.descriptor(), weight.data)
    ids = group_ids.to(device=weight.data.device, dtype=torch.int32).contiguous()
    bad = ((ids < 0) | (ids >= experts)).nonzero()
    if bad.numel():
        raise EreduError(f"native grouped expert {int(ids[int(bad[0])].item())} is outside 0..{experts}")
    routes = ids.numel()
    sorted_ids = bool((ids[1:] >= ids[:-1]).all().item()) if routes > 1 else True
    x = input.contiguous()
    y = torch.empty((routes, N), dtype=torch.bfloat16, device=x.device)
    check(
        _native.lib().eq_gguf_grouped_linear(
            y.data_ptr(), x.data_ptr(), weight.data.contiguous().data_ptr(), weight.data.numel(), int(ty), experts,
            N, K, ids.data_ptr(), routes, int(weight.endian), _native.EQ_DTYPE_BF16, sorted_ids,
            torch.cuda.current_stream().cuda_stream,
        )
    )
    return y


def linear(x: torch.Tensor, desc: TensorDescriptor, raw: torch.Tensor, endian: Endian = Endian.Little) -> torch.Tensor:
    """y = x . W^T with W the GGUF tensor of ``desc`` decoded by the native
    definition, straight from its Q4_K, Q5_K, Q6_K, Q5_1 or Q8_0 blocks (no
    affine expansion): NativeQuantizedTensor::linear with transpose = true
    (safemlx/src/native_quantization.rs:741-772); C ABI eq_gguf_linear.
    x is bf16 [..., K] on the GPU; W's MLX shape is [N, K]."""
    ty = _device_type(desc)
    if not ty.has_device_linear():
        raise EreduError(f"tensor '{desc.name}': no native linear for GGML type {int(ty)} "
                         f"(Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS)")
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


@dataclasses.dataclass
class NativeTensor:
    """A GGML tensor kept in its checkpoint-native blocks on the device: the
    reference's IQuantTensor (convert.rs:26-56) as safemlx hands it to
    NativeQuantizedTensor (safemlx/src/native_quantization.rs:741-772).
    ``shape`` is the logical MLX shape, ``data`` the raw blocks (uint8, GPU)."""

    name: str
    shape: List[int]
    ggml_type: GgmlType
    endian: Endian
    data: torch.Tensor

    def descriptor(self) -> TensorDescriptor:
        return TensorDescriptor(self.name, list(reversed(self.shape)), self.ggml_type, self.data.numel())

    def packed_shape(self) -> List[int]:
        """Rows of packed block bytes (convert.rs:176-194 iquant_packed_shape)."""
        values, nbytes = GgmlType(self.ggml_type).block_and_bytes()
        if not self.shape or self.shape[-1] % values != 0:
            raise EreduError(f"tensor '{self.name}': row width is not divisible by block length {values}")
        return list(self.shape[:-1]) + [self.shape[-1] // values * nbytes]

    def dequantize_f32(self) -> torch.Tensor:
        """IQuantTensor::dequantize_f32 (convert.rs:43-56): for the non-IQ
        encodings the affine route, convert_affine then AffineTensor::dequantize;
        IQ4_NL / IQ4_XS decode factor x level (iquant.rs:271-301)."""
        return dequantize(self.descriptor(), self.data, self.endian, DequantDefinition.Affine, torch.float32)

    def dequantize(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """NativeQuantizedTensor::dequantize: the native decoders
        (safemlx/src/native_quantization.rs:3417-3542)."""
        return dequantize(self.descriptor(), self.data, self.endian, DequantDefinition.Native, dtype)

    def embedding(self, indices: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """NativeQuantizedTensor::embedding (native_quantization.rs:774-789):
        rows ``indices`` decoded by the native definition."""
        return embedding(indices, self.descriptor(), self.data, self.endian, dtype)

    def linear(self, x: torch.Tensor, transpose: bool = True) -> torch.Tensor:
        """NativeQuantizedTensor::linear (native_quantization.rs:741-772): y = x . W^T
        from the blocks (transpose = true, the only form QuantizedLinear uses)."""
        if not transpose:
            raise EreduError("native GGUF linear is implemented for transpose = true")
        return linear(x, self.descriptor(), self.data, self.endian)


@dataclasses.dataclass
class MxFp4Tensor:
    """convert.rs:73-79: E2M1 codes packed 8 per u32 (LSB first) and one E8M0
    scale byte per 32 values, both on the GPU (int32 / uint8 tensors)."""

    weight_shape: List[int]
    scale_shape: List[int]
    weights: torch.Tensor
    scales: torch.Tensor

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """2^(e - 127) * e2m1(code) per value, written as ``dtype``."""
        from .quantization import QuantizationMode, dequantize_with_mode

        rows = self.scales.numel() // self.scale_shape[-1] if self.scale_shape else 1
        out = dequantize_with_mode(self.weights.view(rows, -1), self.scales.view(rows, -1), None, 32, 4,
                                   QuantizationMode.MxFp4, dtype=dtype)
        return out.view(*self.weight_shape[:-1], -1)


def convert_mxfp4(desc: TensorDescriptor, raw: torch.Tensor) -> MxFp4Tensor:
    """Type-39 blocks -> MLX MXFP4 pair, byte-identical to the reference's
    mxfp4 conversion (convert.rs:197-212 shapes, 247-276 packing); either byte
    order (single bytes only).  C ABI eq_gguf_convert_mxfp4."""
    if int(desc.ggml_type) != int(GgmlType.MXFP4):
        raise EreduError(f"tensor '{desc.name}': not an MXFP4 tensor")
    _check_raw(desc, raw)
    shape = desc.mlx_shape()
    if not shape:
        raise EreduError(f"tensor '{desc.name}': MXFP4 scalar is invalid")
    cols = shape[-1]
    if cols % 32 != 0:
        raise EreduError(f"tensor '{desc.name}': MXFP4 row width is not divisible by 32")
    rows = 1
    for d in shape[:-1]:
        rows *= d
    dev = raw.device
    weights = torch.empty((rows, cols // 8), dtype=torch.int32, device=dev)
    scales = torch.empty((rows, cols // 32), dtype=torch.uint8, device=dev)
    check(
        _native.lib().eq_gguf_convert_mxfp4(
            weights.data_ptr(), scales.data_ptr(), raw.contiguous().data_ptr(), raw.numel(), rows, cols,
            torch.cuda.current_stream().cuda_stream,
        )
    )
    weight_shape = shape[:-1] + [cols // 8]
    scale_shape = shape[:-1] + [cols // 32]
    return MxFp4Tensor(weight_shape, scale_shape, weights.view(*weight_shape), scales.view(*scale_shape))


@dataclasses.dataclass
class DenseTensor:
    """A dense GGUF tensor (convert.rs:19-24) on the device, in its MLX shape."""

    name: str
    array: torch.Tensor


def convert(desc: TensorDescriptor, raw: torch.Tensor, endian: Endian = Endian.Little):
    """eredu_gguf's convert (convert.rs:276-313) on device payloads, routed by
    ``conversion_kind``: a DenseTensor (dense types), a NativeTensor (blocks
    kept as stored: little-endian Q4_K / Q5_K / Q6_K / Q5_1 / Q8_0), an
    MxFp4Tensor (type 39), or an AffineTensor (Q4_0, Q4_1, Q5_0, Q2_K, Q3_K in
    either byte order; the natively executed types in big-endian files).
    Encodings without device kernels (the IQ types) are refused with the type
    named."""
    if raw.dtype != torch.uint8 or not raw.is_cuda:
        raise EreduError("raw GGUF payload must be a uint8 tensor on the GPU")
    if raw.numel() != desc.byte_len:
        raise EreduError(f"tensor '{desc.name}': payload length does not match descriptor")
    ty = ggml_type_from_code(int(desc.ggml_type))
    kind = conversion_kind(ty, endian)
    if kind.kind == "dense":
        width = ty.block_and_bytes()[1]
        if Endian(endian) == Endian.Big and width > 1:  # normalize_dense (convert.rs:216-233): swap each element
            raw = raw.view(-1, width).flip(-1).contiguous().view(-1)
        return DenseTensor(desc.name, raw.view(kind.dtype).reshape(desc.mlx_shape()))
    if kind.kind == "native":
        if not ty.has_device_linear():
            raise EreduError(f"tensor '{desc.name}': GGML type {int(ty)} stays native in eredu, and this library "
                             f"executes only Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS blocks")
        shape = desc.mlx_shape()
        values, _ = ty.block_and_bytes()
        if not shape or shape[-1] % values != 0:
            raise EreduError(f"tensor '{desc.name}': row width is not divisible by block length {values}")
        return NativeTensor(desc.name, shape, ty, Endian(endian), raw)
    if kind.kind == "mxfp4":
        return convert_mxfp4(desc, raw)
    return convert_affine(desc, raw, endian)
