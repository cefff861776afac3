"""The quantized-linear dispatch on the GPU: GGUF routing (little-endian
Q4_K / Q8_0 stay native, the rest become affine), QuantizedLinear's native
and affine branches, the layer factory for each WeightQuantization, and
QuantizedEmbedding -- each against the oracle of the definition it must
follow (safemlx/src/nn/quantized.rs:394-435,787-835;
eredu/src/backend/mlx/nn/linear.rs:64-101; eredu-gguf/src/convert.rs:125-140)."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError, QuantizedEmbedding, QuantizedLinear
from eredu_amd import gguf as G
from eredu_amd import gguf_file as F
from eredu_amd import nn
from eredu_amd.checkpoint import WeightQuantization
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_u8, dev_words, host_bits16, host_f32, synthetic_blocks, synthetic_linear

pytestmark = pytest.mark.gpu


def swap_f16_headers(ty, raw):
    """The same blocks stored big-endian (f16 d, and Q4_K's dmin, byte-swapped)."""
    _, nbytes = G.GgmlType(ty).block_and_bytes()
    b = raw.reshape(-1, nbytes).copy()
    for h in ([0, 2] if ty == G.GgmlType.Q4K else [0]):
        b[:, [h, h + 1]] = b[:, [h + 1, h]]
    return b.reshape(-1)


def x_bits(M, K, seed):
    return orc.f32_to_bf16_bits(np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32))


def native_ref(ty, raw, N, K, xb, definition):
    W = orc.gguf_dequant_f32(int(ty), raw, int(definition)).reshape(N, K).astype(np.float64)
    return orc.bf16_bits_to_f32(xb).astype(np.float64) @ W.T


@pytest.mark.parametrize("endian", ["little", "big"])
def test_streamed_q4k_and_q8_0_follow_eredus_routing(cuda, tmp_path, endian):
    """A streamed little-endian Q4_K / Q8_0 tensor stays in its blocks and its
    layer computes with the native definition; big-endian ones and Q4_0 are
    expanded to the affine triple (and compute with the affine definition)."""
    print(f"[case] routed stream endian={endian}", flush=True)
    N, K = 96, 1024
    spec = [("blk.0.ffn_down.weight", G.GgmlType.Q4K), ("blk.0.ffn_up.weight", G.GgmlType.Q8_0),
            ("blk.0.attn_q.weight", G.GgmlType.Q4_0)]
    raws, tensors = {}, []
    for i, (name, ty) in enumerate(spec):
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), N * K // vals, seed=40 + i)
        raws[name] = raw
        stored = swap_f16_headers(ty, raw) if endian == "big" else raw
        tensors.append((name, [K, N], int(ty), stored.tobytes()))
    path = tmp_path / "m.gguf"
    with open(path, "wb") as f:
        F.write_gguf(f, {}, tensors, endian=endian)
    out = F.stream_convert(str(path), staging_bytes=8192)
    xb = x_bits(3, K, 5)
    for name, ty in spec:
        t = out[name]
        native = endian == "little" and ty in (G.GgmlType.Q4K, G.GgmlType.Q8_0)
        if native:
            assert isinstance(t, G.NativeTensor) and t.shape == [N, K]
            assert t.packed_shape() == [N, K // ty.block_and_bytes()[0] * ty.block_and_bytes()[1]]
            layer = QuantizedLinear.from_native(t)
            y = layer(dev_bf16(xb))
            # bit for bit the native linear kernel, within the matmul rule of the native definition
            y_direct = G.linear(dev_bf16(xb), t.descriptor(), t.data, t.endian)
            assert torch.equal(y.view(torch.int16), y_direct.view(torch.int16))
            ref = native_ref(ty, raws[name], N, K, xb, G.DequantDefinition.Native)
            ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=True)
            assert ok, f"{name}: {worst:.3e}"
            # the dense decode is the native definition, which for Q4_K is not the affine one
            dense = host_bits16(t.dequantize(torch.bfloat16)).reshape(-1)
            nat = orc.gguf_dequant_bf16(int(ty), raws[name], int(G.DequantDefinition.Native))
            aff = orc.gguf_dequant_bf16(int(ty), raws[name], int(G.DequantDefinition.Affine))
            assert np.array_equal(dense, nat)
            if ty == G.GgmlType.Q4K:
                assert not np.array_equal(nat, aff)
        else:
            assert isinstance(t, G.AffineTensor)
            w, s, b = orc.gguf_convert_affine(int(ty), raws[name])
            assert np.array_equal(t.weights.cpu().numpy().view(np.uint32).reshape(-1), w)
            layer = QuantizedLinear(t.weights, t.scales, t.biases, t.group_size, t.bits)
            y = layer(dev_bf16(xb))
            ref = orc.quantized_matmul_f64(xb, orc.BF16, w.reshape(N, -1), s.reshape(N, -1), b.reshape(N, -1),
                                           orc.F16, True, t.group_size, t.bits, N, K)
            ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=True)
            assert ok, f"{name}: {worst:.3e}"


def test_layer_factory_native_gguf(cuda):
    """LinearSpec with GgufIQuant -> unloaded_iq; loaded block rows run the
    native linear (plus the dense bias)."""
    N, K = 64, 512
    ty = G.GgmlType.Q4K
    layer = nn.linear(nn.LinearSpec(K, N, True, "blk.0.attn_o.weight", WeightQuantization.GgufIQuant(int(ty))))
    assert isinstance(layer, QuantizedLinear) and layer.native_format == ty
    assert tuple(layer.weight.shape) == (N, K // 256 * 144) and layer.weight.dtype == torch.uint8
    assert (layer.group_size, layer.bits, layer.input_dims) == (256, 144, K)
    raw = synthetic_blocks(int(ty), N * K // 256, seed=9)
    bias = torch.linspace(-1, 1, N, device="cuda", dtype=torch.float32)
    layer.load_parameters({"weight": dev_u8(raw).view(N, -1), "bias": bias})
    xb = x_bits(2, K, 1)
    y = layer(dev_bf16(xb))
    assert y.dtype == torch.float32  # bf16 product + f32 bias promotes, as MLX's add does
    ref = native_ref(ty, raw, N, K, xb, G.DequantDefinition.Native) + bias.cpu().numpy().astype(np.float64)
    base = native_ref(ty, raw, N, K, xb, G.DequantDefinition.Native)
    err = np.abs(y.cpu().numpy() - ref)
    rms = float(np.sqrt(np.mean(base ** 2)))
    assert np.all(err <= 1e-2 * rms + orc.bf16_half_ulp(base) + 1e-6)
    with pytest.raises(EreduError, match="shape"):
        layer.load_parameters({"weight": torch.zeros((N, 10), dtype=torch.uint8, device="cuda")})


@pytest.mark.parametrize("quant", [None, WeightQuantization.Affine(64, 4), WeightQuantization.Affine(32, 8)])
def test_layer_factory_affine_and_dense(cuda, quant):
    N, K = 128, 512
    layer = nn.linear(nn.LinearSpec(K, N, False, "w", quant))
    xb = x_bits(4, K, 2)
    if quant is None:
        assert isinstance(layer, nn.Linear) and layer.shape() == (N, K) and layer.weight.dtype == torch.float32
        return
    assert isinstance(layer, QuantizedLinear)
    assert tuple(layer.weight.shape) == (N, K * quant.bits // 32) and layer.scales.dtype == torch.float32
    # the f32 placeholders are usable as they are (zeros give zeros) ...
    assert torch.count_nonzero(layer(dev_bf16(xb)).float()).item() == 0
    # ... and load the checkpoint's parameters in place
    w, s, b = synthetic_linear(N, K, quant.group_size, quant.bits, seed=3)
    layer.load_parameters({"weight": dev_words(w), "scales": dev_bf16(s), "biases": dev_bf16(b)})
    y = layer(dev_bf16(xb))
    ref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, orc.BF16, True, quant.group_size, quant.bits, N, K)
    assert orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=True)[0]


def test_quantized_embedding_affine_and_native(cuda):
    V, D = 200, 256
    w, s, b = synthetic_linear(V, D, 64, 4, seed=4)
    emb = QuantizedEmbedding(dev_words(w), dev_bf16(s), dev_bf16(b), 64, 4)
    ids = torch.tensor([[3, 199, 0], [57, 3, 120]], dtype=torch.int32, device="cuda")
    rows = emb(ids)
    assert tuple(rows.shape) == (2, 3, D) and rows.dtype == torch.bfloat16
    ref = orc.affine_dequant_f32(w, s, b, orc.BF16, V, D, 64, 4)
    flat = ids.cpu().numpy().reshape(-1)
    assert np.array_equal(host_bits16(rows).reshape(len(flat), D), orc.f32_to_bf16_bits(ref[flat]))
    # tied output projection
    xb = x_bits(2, D, 6)
    y = emb.as_linear(dev_bf16(xb))
    yref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, orc.BF16, True, 64, 4, V, D)
    assert orc.matmul_within_tolerance(host_f32(y), yref, out_is_bf16=True)[0]
    # native Q8_0 rows: NativeQuantizedTensor::embedding (native_quantization.rs:915-939),
    # float32 rows of the native decoder, and the reference's range error
    raw = synthetic_blocks(8, V * D // 32, seed=8)
    nt = G.NativeTensor("tok_embd.weight", [V, D], G.GgmlType.Q8_0, G.Endian.Little, dev_u8(raw))
    nemb = QuantizedEmbedding.from_native(nt)
    out = nemb(ids)
    assert tuple(out.shape) == (2, 3, D) and out.dtype == torch.float32
    dense = orc.gguf_dequant_f32(8, raw, int(G.DequantDefinition.Native)).reshape(V, D)
    assert np.array_equal(out.cpu().numpy().reshape(len(flat), D).view(np.uint32), dense[flat].view(np.uint32))
    with pytest.raises(EreduError, match="outside 0..200"):
        nemb(torch.tensor([5, 200], dtype=torch.int32, device="cuda"))
