"""eredu_amd -- MI355X (gfx950) quantized-linear hot path.

Group-wise affine quantized matmul (qmv for decode, qmm for prefill) and the
GGUF Q4_0 / Q8_0 / Q4_K block dequant and convert that feeds it, as
hand-written HIP kernels behind a C ABI (``include/eredu_hip.h``), with a
host-side mirror of the reference's operator API:

* :mod:`eredu_amd.quantization` -- safemlx ``quantized_matmul[_with_mode]``,
  ``gather_qmm[_with_mode]``, ``dequantize[_with_mode]``,
  ``quantize[_with_mode]``, ``QuantizedLinear``.
* :mod:`eredu_amd.gguf` -- eredu-gguf ``conversion_kind`` routing, ``convert``,
  ``convert_affine`` / ``AffineTensor``, ``NativeTensor`` (blocks kept as
  stored), dense dequantization and the native Q4_K / Q5_K / Q6_K / Q5_1 /
  Q8_0 linear.
* :mod:`eredu_amd.nn` -- the linear-layer dispatch (``LinearSpec`` ->
  dense ``Linear`` or ``QuantizedLinear`` for affine / MXFP4 / native GGUF).
* :mod:`eredu_amd.checkpoint` -- MLX-LM quantized SafeTensors checkpoints.
* :mod:`eredu_amd.gguf_file` -- GGUF container reader/writer and the
  streaming load into the device-side convert.
* :mod:`eredu_amd.decode` -- the Llama decode step around the projections.
"""
from ._native import EreduError
from .quantization import (
    DEFAULT_BITS,
    DEFAULT_GROUP_SIZE,
    QuantizationMode,
    QuantizedEmbedding,
    QuantizedLinear,
    dequantize,
    dequantize_with_mode,
    gather_qmm,
    gather_qmm_with_mode,
    quantized_matmul,
    quantized_matmul_batched,
    quantized_matmul_with_mode,
    quantized_packed_dimension,
    quantize,
    quantize_with_mode,
)

__all__ = [
    "EreduError",
    "DEFAULT_BITS",
    "DEFAULT_GROUP_SIZE",
    "QuantizationMode",
    "QuantizedEmbedding",
    "QuantizedLinear",
    "dequantize",
    "dequantize_with_mode",
    "gather_qmm",
    "gather_qmm_with_mode",
    "quantized_matmul",
    "quantized_matmul_batched",
    "quantized_matmul_with_mode",
    "quantized_packed_dimension",
    "quantize",
    "quantize_with_mode",
]
