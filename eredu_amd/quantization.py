"""Host-side mirror of safemlx's quantization operators on the gfx950 kernels.

Names, defaults, argument meaning and error behaviour follow
``safemlx/src/ops/quantization.rs`` (the drop-in boundary eredu's
``QuantizedLinear`` calls) and ``safemlx/src/nn/quantized.rs``.  Tensors are
torch tensors on the GPU (PyTorch is used only for device memory and streams);
all arithmetic runs in the HIP library through the C ABI.  Packed weights are
u32 words; torch.int32 / torch.uint32 tensors are accepted as their bit
containers.
"""
from __future__ import annotations

import enum
from typing import List, Optional, Sequence, Tuple

import torch

from . import _native
from ._native import EreduError, check

DEFAULT_GROUP_SIZE = 64  # safemlx/src/ops/quantization.rs:11
DEFAULT_BITS = 4  # safemlx/src/ops/quantization.rs:12

_DTYPE_CODE = {
    torch.float32: _native.EQ_DTYPE_F32,
    torch.float16: _native.EQ_DTYPE_F16,
    torch.bfloat16: _native.EQ_DTYPE_BF16,
}
_WORD_DTYPES = (torch.int32, getattr(torch, "uint32", torch.int32))


class QuantizationMode(enum.Enum):
    """safemlx/src/ops/quantization.rs:16-46."""

    Affine = "affine"
    MxFp4 = "mxfp4"

    def has_biases(self) -> bool:
        return self is QuantizationMode.Affine

    def validate(self, group_size: int, bits: int) -> None:
        if self is QuantizationMode.MxFp4 and (group_size != 32 or bits != 4):
            raise EreduError(
                f"MXFP4 requires group_size=32 and bits=4, got group_size={group_size} bits={bits}"
            )


def quantized_packed_dimension(dimension: int, bits: int) -> int:
    """Number of u32 words per packed row (safemlx/src/ops/quantization.rs:62-64)."""
    return dimension * bits // 32


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise EreduError(f"{what} must be float32, float16 or bfloat16, got {t.dtype}") from None


def _require_device(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise EreduError("all arrays must live on the GPU (the library has no host path)")


def _scale_code(scales: torch.Tensor, mode: "QuantizationMode") -> int:
    """Affine scales are float32/float16/bfloat16; MXFP4 scales are E8M0
    bytes (uint8, quantized.rs:240-244)."""
    if mode is QuantizationMode.MxFp4:
        if scales.dtype != torch.uint8:
            raise EreduError(f"MXFP4 scales must be uint8 E8M0 bytes, got {scales.dtype}")
        return _native.EQ_DTYPE_U8
    return _dtype_code(scales, "scales")


def _check_biases(biases: Optional[torch.Tensor], mode: "QuantizationMode") -> None:
    if mode is QuantizationMode.MxFp4 and biases is not None:
        raise EreduError("MXFP4 has no biases")


def _words(w: torch.Tensor) -> torch.Tensor:
    if w.dtype not in _WORD_DTYPES:
        raise EreduError(f"quantized weights must be packed u32 words, got {w.dtype}")
    return w


def quantized_matmul_with_mode(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor],
    transpose: bool,
    group_size: int,
    bits: int,
    mode: QuantizationMode = QuantizationMode.Affine,
) -> torch.Tensor:
    """Quantized matmul with an explicit encoding
    (safemlx/src/ops/quantization.rs:190-226; C ABI: eq_quantized_matmul).

    transpose=True : w [N, K*bits/32], scales/biases [N, K/gs], y = x @ W^T.
    transpose=False: w [K, N*bits/32], scales/biases [K, N/gs], y = x @ W.
    x [..., K] -> y [..., N] in x's dtype.

    With batch dimensions on w (w [..., rows, cols], as the quantized KV
    attention of eredu/src/backend/mlx/nn/tensor.rs:76-150 passes them), x is
    [..., M, K] and the two batch shapes broadcast: y[b] = x[b] @ W[b] (MLX's
    rule), computed by eq_gather_qmm with the broadcast batch indices.
    """
    mode.validate(group_size, bits)
    _check_biases(biases, mode)
    if w.dim() > 2:
        if x.dim() < 2:
            raise EreduError("with batched weights, x must be at least [M, K]")
        try:
            torch.broadcast_shapes(tuple(x.shape[:-2]), tuple(w.shape[:-2]))
        except RuntimeError as e:
            raise EreduError(f"batch dimensions of x {tuple(x.shape[:-2])} and w {tuple(w.shape[:-2])} "
                             f"do not broadcast") from e
        return gather_qmm_with_mode(x, w, scales, biases, None, None, transpose, group_size, bits, False, mode)
    N, K = _check_operands(x, w, scales, biases, transpose, group_size, bits)
    x_code = _dtype_code(x, "x")
    s_code = _scale_code(scales, mode)
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    w = w.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous() if biases is not None else None
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    check(
        _native.lib().eq_quantized_matmul(
            y.data_ptr(), x2.data_ptr(), w.data_ptr(), scales.data_ptr(),
            biases.data_ptr() if biases is not None else None,
            M, N, K, bool(transpose), int(group_size), int(bits), mode.value.encode(), x_code, s_code, _stream(),
        )
    )
    return y.reshape(*x.shape[:-1], N)


def quantized_matmul(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor] = None,
    transpose: bool = False,
    group_size: int = DEFAULT_GROUP_SIZE,
    bits: int = DEFAULT_BITS,
) -> torch.Tensor:
    """Affine quantized matmul with safemlx's defaults (transpose=False, gs 64,
    bits 4; safemlx/src/ops/quantization.rs:165-184)."""
    return quantized_matmul_with_mode(x, w, scales, biases, transpose, group_size, bits, QuantizationMode.Affine)


def _check_operands(x, w, scales, biases, transpose, group_size, bits):
    """Shape/dtype rules of quantized_matmul_with_mode; returns (N, K)."""
    _require_device(x, w, scales, biases)
    _words(w)
    if w.dim() != 2 or scales.dim() != 2:
        raise EreduError("w and scales must be 2-D")
    if bits not in (2, 3, 4, 5, 6, 8):
        raise EreduError(f"bits must be one of 2, 3, 4, 5, 6, 8, got {bits}")
    if transpose:
        N, K = w.shape[0], w.shape[1] * 32 // bits
    else:
        K, N = w.shape[0], w.shape[1] * 32 // bits
    if x.shape[-1] != K:
        raise EreduError(
            f"shapes {tuple(x.shape)} and {tuple(w.shape)} are incompatible for quantized matmul "
            f"(x's last dimension must be {K})"
        )
    packed_dim = K if transpose else N
    if group_size <= 0 or packed_dim % group_size != 0:
        raise EreduError(f"the quantized dimension {packed_dim} is not divisible by group_size {group_size}")
    expect_scales = (w.shape[0], packed_dim // group_size)
    if tuple(scales.shape) != expect_scales:
        raise EreduError(f"scales has shape {tuple(scales.shape)}, expected {expect_scales}")
    if biases is not None and (tuple(biases.shape) != expect_scales or biases.dtype != scales.dtype):
        raise EreduError("biases must match scales in shape and dtype")
    return N, K


def quantized_matmul_batched(
    problems: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]],
    transpose: bool = True,
    group_size: int = DEFAULT_GROUP_SIZE,
    bits: int = DEFAULT_BITS,
    mode: QuantizationMode = QuantizationMode.Affine,
) -> List[torch.Tensor]:
    """Several independent quantized matmuls ``(x, w, scales, biases)`` that share
    the encoding and the activation row count, e.g. the q/k/v projections of one
    decoder layer (eredu-architectures/src/llama.rs:272-295).  Returns the same
    tensors as one quantized_matmul_with_mode call per problem, bit for bit
    (C ABI: eq_quantized_matmul_batched), from as few kernel launches as the
    device path allows."""
    mode.validate(group_size, bits)
    if not problems:
        return []
    x0, _, s0, _ = problems[0]
    x_code, s_code = _dtype_code(x0, "x"), _scale_code(s0, mode)
    keep, outs = [], []
    arr = (_native.QmmProblem * len(problems))()
    M = None
    for i, (x, w, scales, biases) in enumerate(problems):
        _check_biases(biases, mode)
        N, K = _check_operands(x, w, scales, biases, transpose, group_size, bits)
        if x.dtype != x0.dtype or scales.dtype != s0.dtype:
            raise EreduError("all problems of a batch must share the activation and scale dtypes")
        x2 = x.reshape(-1, K).contiguous()
        if M is None:
            M = x2.shape[0]
        elif x2.shape[0] != M:
            raise EreduError("all problems of a batch must have the same number of activation rows")
        w, scales = w.contiguous(), scales.contiguous()
        biases = biases.contiguous() if biases is not None else None
        y = torch.empty((M, N), dtype=x.dtype, device=x.device)
        keep += [x2, w, scales, biases]
        outs.append((y, x.shape[:-1], N))
        arr[i] = _native.QmmProblem(y.data_ptr(), x2.data_ptr(), w.data_ptr(), scales.data_ptr(),
                                    biases.data_ptr() if biases is not None else None, N, K)
    check(
        _native.lib().eq_quantized_matmul_batched(
            arr, len(problems), M, bool(transpose), int(group_size), int(bits), mode.value.encode(), x_code, s_code,
            _stream(),
        )
    )
    return [y.reshape(*lead, N) for y, lead, N in outs]


def gather_qmm_with_mode(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor],
    lhs_indices: Optional[torch.Tensor],
    rhs_indices: Optional[torch.Tensor],
    transpose: bool,
    group_size: int,
    bits: int,
    sorted_indices: bool,
    mode: QuantizationMode = QuantizationMode.Affine,
) -> torch.Tensor:
    """Gathered quantized matmul (safemlx/src/ops/quantization.rs:338-379; C ABI:
    eq_gather_qmm), the routed-expert primitive of
    eredu/src/backend/mlx/nn/moe.rs:121-139.

    x [..., M, K]; w [..., N, K*bits/32] (transpose) or [..., K, N*bits/32];
    scales/biases [..., rows, packed_dim/gs].  lhs_indices index x's batch
    elements (flattened), rhs_indices w's; an absent array is arange over
    that operand's batch shape.  The two broadcast to the output batch shape;
    y [*batch, M, N] with y[b] = quantized_matmul(x[lhs[b]], w[rhs[b]]).
    The indices are read on the device: an out-of-range index gives zero
    output rows.  sorted_indices promises ascending rhs_indices (MLX's
    meaning): with it, many single-row routes run as one MFMA GEMM per
    expert (results equal within the matmul rule).
    """
    mode.validate(group_size, bits)
    _check_biases(biases, mode)
    _require_device(x, w, scales, biases, lhs_indices, rhs_indices)
    _words(w)
    if x.dim() < 2 or w.dim() < 2 or scales.dim() != w.dim():
        raise EreduError("x and w need at least 2 dimensions, scales as many as w")
    xb_shape, wb_shape = tuple(x.shape[:-2]), tuple(w.shape[:-2])
    if tuple(scales.shape[:-2]) != wb_shape or (biases is not None and tuple(biases.shape[:-2]) != wb_shape):
        raise EreduError("scales and biases must have w's batch dimensions")
    x_batches = 1
    for d in xb_shape:
        x_batches *= d
    w_batches = 1
    for d in wb_shape:
        w_batches *= d
    w2 = w.reshape(-1, *w.shape[-2:])
    s2 = scales.reshape(-1, *scales.shape[-2:])
    b2 = biases.reshape(-1, *biases.shape[-2:]) if biases is not None else None
    N, K = _check_operands(x, w2[0], s2[0], b2[0] if b2 is not None else None, transpose, group_size, bits)
    M = x.shape[-2]
    dev = x.device
    if lhs_indices is None:
        lhs_indices = torch.arange(x_batches, device=dev, dtype=torch.int32).reshape(xb_shape)
    if rhs_indices is None:
        rhs_indices = torch.arange(w_batches, device=dev, dtype=torch.int32).reshape(wb_shape)
    for name, idx in (("lhs_indices", lhs_indices), ("rhs_indices", rhs_indices)):
        if idx.dtype.is_floating_point or idx.dtype.is_complex or idx.dtype == torch.bool:
            raise EreduError(f"{name} must be an integer array, got {idx.dtype}")
    try:
        batch_shape = torch.broadcast_shapes(lhs_indices.shape, rhs_indices.shape)
    except RuntimeError as e:
        raise EreduError(f"lhs_indices {tuple(lhs_indices.shape)} and rhs_indices "
                         f"{tuple(rhs_indices.shape)} do not broadcast") from e
    lhs = lhs_indices.to(torch.int32).broadcast_to(batch_shape).contiguous().reshape(-1)
    rhs = rhs_indices.to(torch.int32).broadcast_to(batch_shape).contiguous().reshape(-1)
    batch = lhs.numel()
    x3 = x.reshape(x_batches, M, K).contiguous()
    w2, s2 = w2.contiguous(), s2.contiguous()
    b2 = b2.contiguous() if b2 is not None else None
    y = torch.empty((batch, M, N), dtype=x.dtype, device=dev)
    check(
        _native.lib().eq_gather_qmm(
            y.data_ptr(), x3.data_ptr(), w2.data_ptr(), s2.data_ptr(), b2.data_ptr() if b2 is not None else None,
            lhs.data_ptr(), rhs.data_ptr(), batch, x_batches, w_batches, M, N, K, bool(transpose),
            int(group_size), int(bits), mode.value.encode(), _dtype_code(x, "x"), _scale_code(scales, mode),
            bool(sorted_indices), _stream(),
        )
    )
    return y.reshape(*batch_shape, M, N)


def gather_qmm(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor] = None,
    lhs_indices: Optional[torch.Tensor] = None,
    rhs_indices: Optional[torch.Tensor] = None,
    transpose: bool = True,
    group_size: int = DEFAULT_GROUP_SIZE,
    bits: int = DEFAULT_BITS,
    sorted_indices: bool = False,
) -> torch.Tensor:
    """gather_qmm with safemlx's defaults (transpose=True, gs 64, bits 4,
    affine; safemlx/src/ops/quantization.rs:297-334)."""
    return gather_qmm_with_mode(x, w, scales, biases, lhs_indices, rhs_indices, transpose, group_size, bits,
                                sorted_indices, QuantizationMode.Affine)


def quantize_with_mode(
    w: torch.Tensor,
    group_size: int,
    bits: int,
    mode: QuantizationMode = QuantizationMode.Affine,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """(codes u32-as-int32 [rows, cols * bits / 32], scales, biases) of the
    quantization of w [..., cols] along its last axis
    (safemlx/src/ops/quantization.rs:119-159; C ABI: eq_quantize).  Affine:
    scales and biases in w's dtype.  MXFP4: E2M1 codes, uint8 E8M0 scales
    and no biases (None), as QuantizedArrays.biases is for that mode."""
    mode.validate(group_size, bits)
    _require_device(w)
    cols = w.shape[-1]
    if cols % group_size != 0:
        raise EreduError(f"the last dimension ({cols}) is not divisible by group_size {group_size}")
    w2 = w.reshape(-1, cols).contiguous()
    rows = w2.shape[0]
    wq = torch.empty((rows, cols * bits // 32), dtype=torch.int32, device=w.device)
    mx = mode is QuantizationMode.MxFp4
    scales = torch.empty((rows, cols // group_size), dtype=torch.uint8 if mx else w.dtype, device=w.device)
    biases = None if mx else torch.empty_like(scales)
    check(
        _native.lib().eq_quantize(wq.data_ptr(), scales.data_ptr(), biases.data_ptr() if biases is not None else None,
                                  w2.data_ptr(), rows, cols, int(group_size), int(bits), mode.value.encode(),
                                  _dtype_code(w2, "w"), _stream())
    )
    lead = tuple(w.shape[:-1])
    return (wq.reshape(*lead, -1), scales.reshape(*lead, -1),
            biases.reshape(*lead, -1) if biases is not None else None)


def quantize(w: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE, bits: int = DEFAULT_BITS):
    """Affine quantize with the reference's defaults (quantization.rs:100-117)."""
    return quantize_with_mode(w, group_size, bits, QuantizationMode.Affine)


def dequantize_with_mode(
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor],
    group_size: int,
    bits: int,
    mode: QuantizationMode = QuantizationMode.Affine,
    dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """w_hat = scales * q + biases in the scales' dtype unless ``dtype`` is given
    (safemlx/src/ops/quantization.rs:256-289; C ABI: eq_dequantize).  MXFP4:
    w_hat = 2^(e - 127) * e2m1(q), no biases; the scales being bytes, the
    default output is bfloat16 (MLX's default for its floating-point modes)."""
    mode.validate(group_size, bits)
    _check_biases(biases, mode)
    _require_device(w, scales, biases)
    w = _words(w).contiguous()
    if w.dim() != 2:
        raise EreduError("w must be 2-D")
    rows = w.shape[0]
    cols = w.shape[1] * 32 // bits
    if cols % group_size != 0 or tuple(scales.shape) != (rows, cols // group_size):
        raise EreduError(f"scales has shape {tuple(scales.shape)}, expected {(rows, cols // group_size)}")
    if biases is not None and (tuple(biases.shape) != tuple(scales.shape) or biases.dtype != scales.dtype):
        raise EreduError("biases must match scales in shape and dtype")
    s_code = _scale_code(scales, mode)
    out_dtype = dtype or (torch.bfloat16 if mode is QuantizationMode.MxFp4 else scales.dtype)
    if out_dtype not in _DTYPE_CODE:
        raise EreduError(f"output dtype must be float32, float16 or bfloat16, got {out_dtype}")
    out = torch.empty((rows, cols), dtype=out_dtype, device=w.device)
    scales = scales.contiguous()
    biases = biases.contiguous() if biases is not None else None
    check(
        _native.lib().eq_dequantize(
            out.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr() if biases is not None else None,
            rows, cols, int(group_size), int(bits), mode.value.encode(), s_code, _DTYPE_CODE[out_dtype], _stream(),
        )
    )
    return out


def dequantize(
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: Optional[torch.Tensor] = None,
    group_size: int = DEFAULT_GROUP_SIZE,
    bits: int = DEFAULT_BITS,
) -> torch.Tensor:
    """safemlx/src/ops/quantization.rs:228-254."""
    return dequantize_with_mode(w, scales, biases, group_size, bits, QuantizationMode.Affine)


class QuantizedLinear:
    """Quantized linear layer (safemlx/src/nn/quantized.rs:582-615,787-835).

    Holds either the affine triple -- ``weight`` (packed u32 codes [N, K * bits
    / 32]), ``scales``, ``biases`` -- or checkpoint-native GGML blocks: a
    ``native`` tensor (gguf.NativeTensor), or raw block rows in ``weight``
    (uint8 [N, K / block_values * block_bytes]) with ``native_format`` set.
    ``forward`` dispatches as the reference's does: native -> the native GGUF
    linear; native_format -> the same on the block rows; otherwise
    quantized_matmul(x, weight, scales, biases, transpose=True); then the
    optional dense ``bias`` is added."""

    DEFAULT_GROUP_SIZE = DEFAULT_GROUP_SIZE
    DEFAULT_BITS = DEFAULT_BITS

    def __init__(
        self,
        weight: torch.Tensor,
        scales: Optional[torch.Tensor],
        biases: Optional[torch.Tensor],
        group_size: int = DEFAULT_GROUP_SIZE,
        bits: int = DEFAULT_BITS,
        bias: Optional[torch.Tensor] = None,
        mode: QuantizationMode = QuantizationMode.Affine,
        native=None,
        native_format=None,
        native_endian: int = 0,
        native_columns: int = 0,
    ):
        self.weight = weight
        self.scales = scales
        self.biases = biases
        self.group_size = group_size
        self.bits = bits
        self.bias = bias
        self.mode = mode
        self.native = native
        self.native_format = native_format
        self.native_endian = native_endian
        self.native_columns = native_columns

    # -- construction (quantized.rs:505-580, 621-780) ------------------------

    @classmethod
    def unloaded(cls, input_dims: int, output_dims: int, group_size: int, bits: int, bias: bool,
                 device=None) -> "QuantizedLinear":
        """Placeholder layer carrying only shapes, to be filled by load_parameters
        (quantized.rs:621-640)."""
        return cls.unloaded_with_mode(input_dims, output_dims, group_size, bits, QuantizationMode.Affine, bias,
                                      device)

    @classmethod
    def unloaded_with_mode(cls, input_dims: int, output_dims: int, group_size: int, bits: int,
                           mode: QuantizationMode, bias: bool, device=None) -> "QuantizedLinear":
        """quantized.rs:643-706: u32 weight [out, packed], scales [out, in / gs]
        in f32 (u8 for MXFP4), f32 biases when the mode has them, f32 bias."""
        mode.validate(group_size, bits)
        dev = torch.device("cuda") if device is None else device
        scale_dtype = torch.uint8 if mode is QuantizationMode.MxFp4 else torch.float32
        weight = torch.zeros((output_dims, quantized_packed_dimension(input_dims, bits)), dtype=torch.int32,
                             device=dev)
        scales = torch.zeros((output_dims, input_dims // group_size), dtype=scale_dtype, device=dev)
        biases = (torch.zeros((output_dims, input_dims // group_size), dtype=torch.float32, device=dev)
                  if mode.has_biases() else None)
        b = torch.zeros((output_dims,), dtype=torch.float32, device=dev) if bias else None
        return cls(weight, scales, biases, group_size, bits, b, mode)

    @classmethod
    def unloaded_iq(cls, input_dims: int, output_dims: int, ggml_type, endian, bias: bool,
                    device=None) -> "QuantizedLinear":
        """A layer backed by checkpoint-native GGML block rows (quantized.rs:709-750):
        weight uint8 [out, in / block_values * block_bytes], group_size and bits
        holding the block geometry, scales a [1] placeholder, no biases."""
        from . import gguf as G

        ty = G.ggml_type_from_code(int(ggml_type))
        if not ty.has_native_execution():
            raise EreduError(f"{ty.name} is not an IQ type")
        values, nbytes = ty.block_and_bytes()
        if input_dims <= 0 or input_dims % values != 0:
            raise EreduError(f"IQ linear width {input_dims} is not divisible by {values}")
        dev = torch.device("cuda") if device is None else device
        weight = torch.zeros((output_dims, input_dims // values * nbytes), dtype=torch.uint8, device=dev)
        b = torch.zeros((output_dims,), dtype=torch.float32, device=dev) if bias else None
        return cls(weight, torch.zeros((1,), dtype=torch.float32, device=dev), None, values, nbytes, b,
                   QuantizationMode.Affine, None, ty, int(endian), input_dims)

    @classmethod
    def from_native(cls, native, bias: Optional[torch.Tensor] = None) -> "QuantizedLinear":
        """A layer whose weight is a gguf.NativeTensor (the ``native`` field)."""
        values, nbytes = native.ggml_type.block_and_bytes()
        return cls(native.data.view(native.shape[0], -1), None, None, values, nbytes, bias, QuantizationMode.Affine,
                   native)

    @classmethod
    def try_from_linear(cls, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                        group_size: Optional[int] = None, bits: Optional[int] = None) -> "QuantizedLinear":
        """Quantizes a dense [out, in] weight (quantized.rs:765-780, defaults 64 / 4)."""
        gs = DEFAULT_GROUP_SIZE if group_size is None else group_size
        b = DEFAULT_BITS if bits is None else bits
        w, s, bi = quantize_with_mode(weight, gs, b, QuantizationMode.Affine)
        return cls(w, s, bi, gs, b, bias, QuantizationMode.Affine)

    def load_parameters(self, params: dict) -> None:
        """Replaces placeholders by loaded tensors (``weight``, ``scales``,
        ``biases``, ``bias``), each of the placeholder's shape."""
        for name in ("weight", "scales", "biases", "bias"):
            if name not in params:
                continue
            cur, new = getattr(self, name), params[name]
            if cur is None:
                raise EreduError(f"layer has no parameter {name!r}")
            if tuple(new.shape) != tuple(cur.shape):
                raise EreduError(f"parameter {name!r}: shape {tuple(new.shape)}, expected {tuple(cur.shape)}")
            setattr(self, name, new)

    # -- geometry and forward -------------------------------------------------

    @property
    def output_dims(self) -> int:
        return self.weight.shape[0]

    @property
    def input_dims(self) -> int:
        if self.native is not None:
            return self.native.shape[-1]
        if self.native_format is not None:
            return self.native_columns
        return self.weight.shape[1] * 32 // self.bits

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.native is not None:
            y = self.native.linear(x, True)
        elif self.native_format is not None:
            from . import gguf as G

            nt = G.NativeTensor("<native blocks>", [self.weight.shape[0], self.native_columns], self.native_format,
                                G.Endian(self.native_endian), self.weight.contiguous().view(-1))
            y = nt.linear(x, True)
        else:
            y = quantized_matmul_with_mode(
                x, self.weight, self.scales, self.biases, True, self.group_size, self.bits, self.mode
            )
        if self.bias is not None:
            y = y + self.bias
        return y

    __call__ = forward


class QuantizedEmbedding:
    """Quantized token embedding (safemlx/src/nn/quantized.rs:200-435):
    ``forward`` gathers the rows of the ids (codes, scales, biases) and
    dequantizes them (dequantize_with_mode, output in the scales' dtype), or,
    for native GGML block rows, decodes the gathered blocks with the native
    definition; ``as_linear`` is the tied output projection
    (quantized_matmul with transpose = true, or the native linear)."""

    DEFAULT_GROUP_SIZE = DEFAULT_GROUP_SIZE
    DEFAULT_BITS = DEFAULT_BITS

    def __init__(self, weight: torch.Tensor, scales: Optional[torch.Tensor], biases: Optional[torch.Tensor],
                 group_size: int = DEFAULT_GROUP_SIZE, bits: int = DEFAULT_BITS,
                 mode: QuantizationMode = QuantizationMode.Affine, native=None):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.native = native

    @classmethod
    def unloaded(cls, embedding_count: int, dimensions: int, group_size: int, bits: int,
                 device=None) -> "QuantizedEmbedding":
        """Placeholder table carrying only shapes (quantized.rs:211-227)."""
        return cls.unloaded_with_mode(embedding_count, dimensions, group_size, bits, QuantizationMode.Affine, device)

    @classmethod
    def unloaded_with_mode(cls, embedding_count: int, dimensions: int, group_size: int, bits: int,
                           mode: QuantizationMode, device=None) -> "QuantizedEmbedding":
        """quantized.rs:229-280: u32 codes [count, packed], scales [count,
        dims / gs] in f32 (u8 for MXFP4), f32 biases when the mode has them."""
        mode.validate(group_size, bits)
        dev = torch.device("cuda") if device is None else device
        scale_dtype = torch.uint8 if mode is QuantizationMode.MxFp4 else torch.float32
        weight = torch.zeros((embedding_count, quantized_packed_dimension(dimensions, bits)), dtype=torch.int32,
                             device=dev)
        scales = torch.zeros((embedding_count, dimensions // group_size), dtype=scale_dtype, device=dev)
        biases = (torch.zeros((embedding_count, dimensions // group_size), dtype=torch.float32, device=dev)
                  if mode.has_biases() else None)
        return cls(weight, scales, biases, group_size, bits, mode)

    @classmethod
    def try_from_embedding(cls, table: torch.Tensor, group_size: Optional[int] = None,
                           bits: Optional[int] = None) -> "QuantizedEmbedding":
        gs = DEFAULT_GROUP_SIZE if group_size is None else group_size
        b = DEFAULT_BITS if bits is None else bits
        w, s, bi = quantize_with_mode(table, gs, b, QuantizationMode.Affine)
        return cls(w, s, bi, gs, b)

    @classmethod
    def from_native(cls, native) -> "QuantizedEmbedding":
        values, nbytes = native.ggml_type.block_and_bytes()
        return cls(native.data.view(native.shape[0], -1), None, None, values, nbytes, QuantizationMode.Affine, native)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        if self.native is not None:
            # native_quantization.rs:915-939: float32 rows, ids checked against
            # the table before any device work
            return self.native.embedding(ids, torch.float32)
        flat = ids.reshape(-1).to(torch.int64)
        w = self.weight.index_select(0, flat)
        s = self.scales.index_select(0, flat)
        b = self.biases.index_select(0, flat) if self.biases is not None else None
        out = dequantize_with_mode(w, s, b, self.group_size, self.bits, self.mode)
        return out.reshape(*ids.shape, -1)

    __call__ = forward

    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        if self.native is not None:
            return self.native.linear(x, True)
        return quantized_matmul_with_mode(x, self.weight, self.scales, self.biases, True, self.group_size, self.bits,
                                          self.mode)
