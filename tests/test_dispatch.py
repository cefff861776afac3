"""Host-side dispatch rules (no GPU): GGUF conversion routing, the
WeightQuantization variants and the shapes of unloaded layers, after the
reference's own tables and tests."""
import pytest
import torch

from eredu_amd import EreduError, QuantizedLinear
from eredu_amd import gguf as G
from eredu_amd import nn
from eredu_amd.checkpoint import WeightQuantization
from eredu_amd.quantization import QuantizationMode

T = G.GgmlType


def test_conversion_kind_follows_convert_rs():
    # eredu-gguf/src/convert.rs:125-140 with format.rs:403-428
    for ty in (T.F32, T.F16, T.BF16, T.I8, T.I16, T.I32, T.I64, T.F64):
        for e in G.Endian:
            assert G.conversion_kind(ty, e).kind == "dense"
    assert G.conversion_kind(T.BF16, G.Endian.Little).dtype == torch.bfloat16
    for ty in (T.Q4K, T.Q5K, T.Q6K, T.Q5_1, T.Q8_0):
        assert G.conversion_kind(ty, G.Endian.Little).kind == "native"
        k = G.conversion_kind(ty, G.Endian.Big)
        assert (k.kind, k.bits, k.group_size) == ("affine",) + G.affine_config(ty)
    for ty in (T.IQ2XXS, T.IQ2XS, T.IQ3XXS, T.IQ1S, T.IQ4NL, T.IQ3S, T.IQ2S, T.IQ4XS, T.IQ1M):
        assert G.conversion_kind(ty, G.Endian.Big).kind == "native"  # IQ stays native in either order
    for e in G.Endian:
        k = G.conversion_kind(T.Q4_0, e)
        assert (k.kind, k.bits, k.group_size) == ("affine", 4, 32)
        assert G.conversion_kind(T.MXFP4, e).kind == "mxfp4"
    assert (G.conversion_kind(T.Q2K, 0).bits, G.conversion_kind(T.Q2K, 0).group_size) == (2, 16)
    assert (G.conversion_kind(T.Q3K, 0).bits, G.conversion_kind(T.Q6K, 1).group_size) == (3, 16)
    with pytest.raises(EreduError, match="unsupported GGML tensor type 31"):
        G.ggml_type_from_code(31)


def test_block_geometry_table():
    # format.rs:366-400
    assert T.Q4K.block_and_bytes() == (256, 144) and T.Q8_0.block_and_bytes() == (32, 34)
    assert T.Q4_0.block_and_bytes() == (32, 18) and T.MXFP4.block_and_bytes() == (32, 17)
    assert T.IQ4XS.block_and_bytes() == (256, 136) and T.F64.block_and_bytes() == (1, 8)
    assert [t for t in T if t.has_device_kernels()] == [T.Q4_0, T.Q4_1, T.Q5_0, T.Q5_1, T.Q8_0, T.Q2K, T.Q3K,
                                                        T.Q4K, T.Q5K, T.Q6K, T.IQ4NL, T.IQ4XS]


def test_weight_quantization_variants():
    # eredu-checkpoint/src/lib.rs:140-205
    q = WeightQuantization.GgufIQuant(int(T.Q4K), 1)
    assert (q.group_size, q.bits, q.has_biases, q.gguf_iquant()) == (256, 144, False, (12, 1))
    q.validate()
    assert WeightQuantization.MxFp4().has_biases is False
    assert WeightQuantization.Affine(32, 8).gguf_iquant() is None
    with pytest.raises(EreduError, match="group_size"):
        WeightQuantization.Affine(48, 4)
    with pytest.raises(EreduError, match="no MLX checkpoint metadata"):
        q.to_json()
    with pytest.raises(EreduError, match="unknown quantization mode"):
        WeightQuantization.from_json({"group_size": 64, "bits": 4, "mode": "gguf"})
    assert nn.mlx_quantization_mode(WeightQuantization()) is QuantizationMode.Affine
    assert nn.mlx_quantization_mode(WeightQuantization.MxFp4()) is QuantizationMode.MxFp4
    with pytest.raises(EreduError, match="cannot be produced"):
        nn.mlx_quantization_mode(q)


def test_unloaded_parameters_use_mlx_bit_packing():
    # the reference's test of the same name (safemlx/src/nn/quantized.rs:840-868)
    cpu = torch.device("cpu")
    lin = QuantizedLinear.unloaded(1024, 8, 32, 5, False, cpu)
    assert tuple(lin.weight.shape) == (8, 160) and tuple(lin.scales.shape) == (8, 32)
    q6 = QuantizedLinear.unloaded(1024, 8, 16, 6, False, cpu)
    assert tuple(q6.weight.shape) == (8, 192) and tuple(q6.scales.shape) == (8, 64)
    q2 = QuantizedLinear.unloaded(1024, 8, 16, 2, False, cpu)
    assert tuple(q2.weight.shape) == (8, 64) and tuple(q2.scales.shape) == (8, 64)
    q3 = QuantizedLinear.unloaded(1024, 8, 16, 3, False, cpu)
    assert tuple(q3.weight.shape) == (8, 96) and tuple(q3.scales.shape) == (8, 64)
    # f32 placeholders, biases only for affine, u8 scales for MXFP4 (quantized.rs:650-706)
    assert lin.scales.dtype == torch.float32 and lin.biases.dtype == torch.float32 and lin.bias is None
    mx = QuantizedLinear.unloaded_with_mode(256, 4, 32, 4, QuantizationMode.MxFp4, True, cpu)
    assert mx.scales.dtype == torch.uint8 and mx.biases is None and tuple(mx.bias.shape) == (4,)
    with pytest.raises(EreduError, match="MXFP4 requires"):
        QuantizedLinear.unloaded_with_mode(256, 4, 64, 4, QuantizationMode.MxFp4, False, cpu)


def test_layer_factory_shapes():
    # eredu/src/backend/mlx/nn/linear.rs:64-101
    cpu = torch.device("cpu")
    dense = nn.unloaded_maybe_quantized_linear_with_dtype(512, 64, True, None, torch.bfloat16, cpu)
    assert isinstance(dense, nn.Linear) and dense.shape() == (64, 512) and dense.bias.dtype == torch.bfloat16
    aff = nn.unloaded_maybe_quantized_linear(512, 64, False, WeightQuantization.Affine(64, 4), cpu)
    assert isinstance(aff, QuantizedLinear) and tuple(aff.weight.shape) == (64, 64)
    iq = nn.unloaded_maybe_quantized_linear(512, 64, False, WeightQuantization.GgufIQuant(int(T.Q8_0)), cpu)
    assert iq.native_format == T.Q8_0 and tuple(iq.weight.shape) == (64, 512 // 32 * 34)
    assert iq.input_dims == 512 and tuple(iq.scales.shape) == (1,) and iq.biases is None
    with pytest.raises(EreduError, match="not divisible by 256"):
        nn.unloaded_maybe_quantized_linear(500, 64, False, WeightQuantization.GgufIQuant(int(T.Q4K)), cpu)
    with pytest.raises(EreduError, match="not an IQ type"):
        QuantizedLinear.unloaded_iq(512, 64, int(T.Q4_0), 0, False, cpu)
    spec = nn.LinearSpec(512, 64, False, "blk.0.attn_q.weight", None)
    assert isinstance(nn.linear(spec, cpu), nn.Linear)


def test_native_grouped_linear_rejects_host_input():
    """A host input never reaches eq_gguf_grouped_linear: its pointers would be
    read by the device kernels."""
    bank = G.NativeTensor("blk.0.ffn_up_exps.weight", [2, 128, 256], T.Q4K, G.Endian.Little,
                          torch.zeros(2 * 128 * 256 // 256 * 144, dtype=torch.uint8))
    x = torch.zeros((1, 256), dtype=torch.bfloat16)
    with pytest.raises(EreduError, match="CUDA input"):
        G.native_grouped_linear(x, bank, torch.zeros(1, dtype=torch.int32))
