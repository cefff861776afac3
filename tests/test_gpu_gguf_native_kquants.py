"""Native GGUF linear for Q5_K, Q6_K and Q5_1 (eq_gguf_linear, the encodings
eredu keeps in their blocks besides Q4_K / Q8_0): y = x . W^T straight from
the blocks, against the fp64 product with W from ggml's closed-form decoders
(the unrounded factors the reference's native kernels use;
tests/test_oracle_kquants.py pins those closed forms), within the matmul
rule |y - y_ref| <= 1e-2 RMS(y_ref) + 1/2 ulp_bf16.  Q5_K and Q6_K are also
held to the same rule against the reference's other numerics for them, the
f16-rounded affine decode of its non-Metal row path."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_u8, host_f32, synthetic_blocks, synthetic_x
from tests.test_oracle_kquants import _q5_closed, _q5k_closed, _q6k_closed, _to_big_endian

pytestmark = pytest.mark.gpu

T = G.GgmlType


def closed_form(ty, raw, N, K):
    if ty == T.Q5_1:
        W = _q5_closed(raw, False)
    elif ty == T.Q5K:
        W = _q5k_closed(raw)[0]
    else:
        W = _q6k_closed(raw)[0]
    return W.reshape(N, K)


def run_case(ty, N, K, M, seed, endian=G.Endian.Little, offset=0):
    vals, nbytes = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), N * K // vals, seed=seed)
    stored = _to_big_endian(int(ty), raw) if endian == G.Endian.Big else raw
    buf = torch.zeros(stored.size + 16, dtype=torch.uint8, device="cuda")
    buf[offset:offset + stored.size] = dev_u8(stored)
    desc = G.TensorDescriptor("blk.0.ffn_down.weight", [K, N], ty, stored.size)
    xb = synthetic_x(M, K, seed + 1)
    y = G.linear(dev_bf16(xb), desc, buf[offset:offset + stored.size], endian)
    assert list(y.shape) == [M, N] and y.dtype == torch.bfloat16
    xf = orc.bf16_bits_to_f32(xb).astype(np.float64)
    ref = xf @ closed_form(ty, raw, N, K).T
    got = host_f32(y)
    ok, worst, _ = orc.matmul_within_tolerance(got, ref, True)
    assert ok, (ty.name, N, K, M, endian, worst)
    if ty in (T.Q5K, T.Q6K):
        # The reference's non-Metal route for these two formats decodes rows
        # through IQuantTensor::dequantize_f32, the affine form with d * sc
        # rounded to f16 (safemlx/src/native_quantization.rs:987-1000,
        # eredu-gguf/src/convert.rs:43-56,439-564): the same product must
        # also sit within the matmul rule of that numerics.
        W_aff = orc.gguf_dequant_f32(int(ty), raw, int(G.DequantDefinition.Affine)).reshape(N, K)
        ok, worst, _ = orc.matmul_within_tolerance(got, xf @ W_aff.astype(np.float64).T, True)
        assert ok, ("f16-rounded route", ty.name, N, K, M, endian, worst)


# K: Q5_1 rows of 128 and 129 blocks; Q5_K / Q6_K rows of 5, 16 and 56
# superblocks (8 rows per workgroup up to 64 KB of rows, 4 at K = 14336).
# N = 390 leaves a partial row group (its bytes not a multiple of 16: the
# 2-byte staging path); M = 11 takes two launches (8 + 3).
CASES = [(T.Q5_1, 4096), (T.Q5_1, 4128), (T.Q5K, 1280), (T.Q5K, 4096), (T.Q6K, 1280), (T.Q6K, 4096),
         (T.Q6K, 14336)]


@pytest.mark.parametrize("ty,K", CASES)
@pytest.mark.parametrize("M", [1, 3, 8, 11])
def test_native_linear(cuda, ty, K, M):
    print(f"[case] native {ty.name} N=390 K={K} M={M}", flush=True)
    run_case(ty, 390, K, M, seed=K + M + int(ty))


@pytest.mark.parametrize("ty", [T.Q5_1, T.Q5K, T.Q6K])
def test_native_linear_big_endian_and_unaligned_payload(cuda, ty):
    print(f"[case] native {ty.name} big-endian / offset payload", flush=True)
    run_case(ty, 200, 2048, 2, seed=7, endian=G.Endian.Big)
    run_case(ty, 200, 2048, 1, seed=8, offset=2)


def test_native_q6k_row_longer_than_64k(cuda):
    """One Q6_K row of 400 superblocks (84000 bytes): one row per workgroup
    with LDS raised past 64 KB."""
    print("[case] native Q6K K=102400", flush=True)
    run_case(T.Q6K, 24, 102400, 1, seed=9)


def test_llama_shapes_q6k_down_and_head(cuda):
    """Q4_K_M files store ffn_down (and the output head) as Q6_K: 4096 x 14336
    and a 4096-wide head of 32768 rows, at decode."""
    print("[case] native Q6K 4096x14336 and 32768x4096", flush=True)
    run_case(T.Q6K, 4096, 14336, 1, seed=10)
    run_case(T.Q6K, 32768, 4096, 1, seed=11)


def test_convert_keeps_the_new_native_types_in_blocks(cuda):
    """convert.rs:125-140: little-endian Q5_K / Q6_K / Q5_1 stay native; the
    NativeTensor's linear and dequantize run on the device."""
    for ty in (T.Q5_1, T.Q5K, T.Q6K):
        vals, _ = ty.block_and_bytes()
        N, K = 64, 512
        raw = synthetic_blocks(int(ty), N * K // vals, seed=4)
        nt = G.convert(G.TensorDescriptor("w", [K, N], ty, raw.size), dev_u8(raw), G.Endian.Little)
        assert isinstance(nt, G.NativeTensor) and nt.shape == [N, K]
        xb = synthetic_x(2, K, 5)
        ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ closed_form(ty, raw, N, K).T
        ok, worst, _ = orc.matmul_within_tolerance(host_f32(nt.linear(dev_bf16(xb))), ref, True)
        assert ok, (ty.name, worst)
        dense = nt.dequantize(torch.float32).cpu().numpy().reshape(-1)
        assert np.array_equal(dense.view(np.uint32), orc.gguf_dequant_f32(int(ty), raw, 1).view(np.uint32))


def test_native_linear_refuses_non_native_types(cuda):
    raw = dev_u8(np.zeros(84 * 2, np.uint8))
    with pytest.raises(EreduError, match="no native linear"):
        G.linear(dev_bf16(synthetic_x(1, 256, 0)), G.TensorDescriptor("w", [256, 2], T.Q2K, 168), raw)


def test_streamed_file_of_every_affine_type(cuda, tmp_path):
    """A GGUF file holding each of the seven added types, streamed through
    small pinned buffers: stream_convert keeps the little-endian natives
    (Q5_K, Q6_K, Q5_1) in blocks and expands the rest, each bit for bit;
    stream_convert_affine expands all seven."""
    from eredu_amd import gguf_file as F
    from tests.fixtures import host_bits16

    print("[case] stream every k-quant type", flush=True)
    spec = [(T.Q4_1, 256, 12), (T.Q5_0, 256, 12), (T.Q5_1, 512, 8), (T.Q2K, 512, 6), (T.Q3K, 768, 5),
            (T.Q5K, 512, 7), (T.Q6K, 1024, 9)]
    tensors, raws = [], {}
    for i, (ty, cols, rows) in enumerate(spec):
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), rows * cols // vals, seed=70 + i)
        name = f"blk.{i}.w.weight"
        raws[name] = (ty, cols, rows, raw)
        tensors.append((name, [cols, rows], int(ty), raw.tobytes()))
    path = tmp_path / "k.gguf"
    with open(path, "wb") as f:
        F.write_gguf(f, {}, tensors, alignment=32)
    routed = F.stream_convert(str(path), staging_bytes=4096)
    expanded = F.stream_convert_affine(str(path), staging_bytes=4096)
    for name, (ty, cols, rows, raw) in raws.items():
        w, s, b = orc.gguf_convert_affine(int(ty), raw)
        a = expanded[name]
        assert np.array_equal(a.weights.cpu().numpy().view(np.uint32).reshape(-1), w), name
        assert np.array_equal(host_bits16(a.scales).reshape(-1), s) and np.array_equal(host_bits16(a.biases).reshape(-1), b)
        r = routed[name]
        if ty.has_device_linear():
            assert isinstance(r, G.NativeTensor) and r.shape == [rows, cols]
            assert torch.equal(r.data.cpu(), torch.from_numpy(raw))
        else:
            assert isinstance(r, G.AffineTensor)
            assert np.array_equal(r.weights.cpu().numpy().view(np.uint32).reshape(-1), w), name


def test_native_layer_placeholder_for_q6k(cuda):
    """QuantizedLinear.unloaded_iq (quantized.rs:709-750) for Q6_K block rows,
    filled and run: forward is the native linear."""
    from eredu_amd import QuantizedLinear

    N, K = 48, 1024
    raw = synthetic_blocks(int(T.Q6K), N * K // 256, seed=80)
    lin = QuantizedLinear.unloaded_iq(K, N, int(T.Q6K), 0, False, torch.device("cuda"))
    lin.weight.copy_(dev_u8(raw).view(N, -1))
    xb = synthetic_x(3, K, 81)
    ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ closed_form(T.Q6K, raw, N, K).T
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(lin.forward(dev_bf16(xb))), ref, True)
    assert ok, worst


def native_closed_form(ty, raw, N, K):
    """fp64 W of the native definition for the types with an affine form."""
    from tests.test_oracle import _q4k_closed_form_f64

    if ty == T.Q4K:
        return _q4k_closed_form_f64(raw).astype(np.float64).reshape(N, K)
    if ty == T.Q8_0:
        b = raw.reshape(-1, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64)
        return (d * b[:, 2:].view(np.int8).astype(np.float64)).reshape(N, K)
    return closed_form(ty, raw, N, K)


# Prefill (M > 8): the slice's blocks converted to the affine triple in the
# workspace and multiplied on the matrix cores (4/8-bit directly, 5/6-bit
# through the byte re-pack); M = 12, 17 and 130 leave partial 128-row tiles.
@pytest.mark.parametrize("ty,K", [(T.Q4K, 2048), (T.Q5K, 1024), (T.Q6K, 2048), (T.Q5_1, 1024), (T.Q8_0, 2048)])
@pytest.mark.parametrize("M", [12, 17, 64, 130])
def test_native_linear_prefill(cuda, ty, K, M):
    print(f"[case] native prefill {ty.name} N=384 K={K} M={M}", flush=True)
    N = 384
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), N * K // vals, seed=K + M + int(ty) + 1)
    desc = G.TensorDescriptor("blk.0.ffn_up.weight", [K, N], ty, raw.size)
    xb = synthetic_x(M, K, M)
    y = G.linear(dev_bf16(xb), desc, dev_u8(raw))
    ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ native_closed_form(ty, raw, N, K).T
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, True)
    assert ok, (ty.name, M, worst)
    if ty in (T.Q6K, T.Q4K):  # big-endian blocks
        stored = _to_big_endian(int(ty), raw) if ty == T.Q6K else raw.reshape(-1, 144)[:, [1, 0, 3, 2] + list(range(4, 144))].reshape(-1)
        yb = G.linear(dev_bf16(xb), desc, dev_u8(stored), G.Endian.Big)
        ok, worst, _ = orc.matmul_within_tolerance(host_f32(yb), ref, True)
        assert ok, (ty.name, M, "big", worst)


def test_native_prefill_in_slices(cuda):
    """Q8_0 with more rows than one 128 MiB slice of the re-packed triple
    (28928 rows at K = 4096): two equal slices of 14848 rows (the second
    14592), each writing its columns of y."""
    print("[case] native prefill Q8_0 N=29440 K=4096 M=40", flush=True)
    N, K, M = 29440, 4096, 40
    raw = synthetic_blocks(int(T.Q8_0), N * K // 32, seed=12)
    desc = G.TensorDescriptor("w", [K, N], T.Q8_0, raw.size)
    xb = synthetic_x(M, K, 13)
    y = host_f32(G.linear(dev_bf16(xb), desc, dev_u8(raw)))
    rows = np.concatenate([np.arange(0, 64), np.arange(14800, 14900), np.arange(N - 64, N)])
    Wr = native_closed_form(T.Q8_0, raw.reshape(N, -1)[rows].reshape(-1), len(rows), K)
    ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ Wr.T
    ok, worst, _ = orc.matmul_within_tolerance(y[:, rows], ref, True)
    assert ok, worst
