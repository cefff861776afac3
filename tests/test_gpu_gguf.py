"""Bit-exact parity of the HIP GGUF convert / dequant kernels with the oracle,
the reference's golden vectors and edge blocks, through the C ABI."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_u8, golden_rows, host_bits16, synthetic_blocks

pytestmark = pytest.mark.gpu

TYPES = [G.GgmlType.Q4_0, G.GgmlType.Q8_0, G.GgmlType.Q4K]
ROWS, COLS = 4096, 14336  # config-4 MLX shape (GGUF ne0 = 14336, ne1 = 4096)


def desc_for(ty, rows, cols):
    vals, nbytes = ty.block_and_bytes()
    return G.TensorDescriptor("t.weight", [cols, rows], ty, rows * cols // vals * nbytes)


def words_bytes(t):
    return t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32)


def check_convert(ty, raw, rows, cols, endian=G.Endian.Little):
    desc = desc_for(ty, rows, cols)
    a = G.convert_affine(desc, dev_u8(raw), endian)
    torch.cuda.synchronize()
    w, s, b = orc.gguf_convert_affine(int(ty), raw, big_endian=endian == G.Endian.Big)
    bits, gs = G.affine_config(ty)
    assert a.weight_shape == [rows, cols * bits // 32] and a.scale_shape == [rows, cols // gs]
    assert np.array_equal(words_bytes(a.weights).reshape(-1), w), "weights"
    assert np.array_equal(host_bits16(a.scales).reshape(-1), s), "scales"
    assert np.array_equal(host_bits16(a.biases).reshape(-1), b), "biases"
    return a


def check_dense(ty, raw, rows, cols, definition, endian=G.Endian.Little):
    desc = desc_for(ty, rows, cols)
    ref32 = orc.gguf_dequant_f32(int(ty), raw, int(definition), big_endian=endian == G.Endian.Big)
    out = G.dequantize(desc, dev_u8(raw), endian, definition, torch.bfloat16)
    assert list(out.shape) == [rows, cols]
    got16, ref16 = host_bits16(out).reshape(-1), orc.f32_to_bf16_bits(ref32)
    nan16 = lambda v: ((v & 0x7F80) == 0x7F80) & ((v & 0x7F) != 0)  # noqa: E731
    # Bit-exact; a NaN (only from inf * 0 when f16(d*sc) overflows) matches any
    # NaN, since the sign of the default NaN differs between x86 and the GPU.
    assert np.all((got16 == ref16) | (nan16(got16) & nan16(ref16))), "bf16 dense"
    out32 = G.dequantize(desc, dev_u8(raw), endian, definition, torch.float32)
    got = out32.cpu().numpy().reshape(-1)
    assert np.all((got.view(np.uint32) == ref32.view(np.uint32)) | (np.isnan(got) & np.isnan(ref32))), "f32 dense"


@pytest.mark.parametrize("ty", TYPES)
def test_golden_rows_on_device(cuda, ty):
    row = golden_rows()[int(ty)]
    raw = np.frombuffer(row["raw"], dtype=np.uint8).copy()
    vals, _ = ty.block_and_bytes()
    a = G.convert_affine(desc_for(ty, 2, vals), dev_u8(raw))
    torch.cuda.synchronize()
    assert words_bytes(a.weights).tobytes() == row["weight"]
    assert host_bits16(a.scales).tobytes() == row["scales"]
    assert host_bits16(a.biases).tobytes() == row["biases"]
    deq = a.dequantize(torch.float32).cpu().numpy().reshape(-1)
    expected = np.frombuffer(row["dequantized"], dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(deq.astype(np.float16).astype(np.float32), expected)


@pytest.mark.parametrize("ty", TYPES)
def test_convert_full_size_bit_exact(cuda, ty):
    vals, _ = ty.block_and_bytes()
    print(f"[case] convert {ty.name} {ROWS}x{COLS}", flush=True)
    raw = synthetic_blocks(int(ty), ROWS * COLS // vals, seed=int(ty))
    check_convert(ty, raw, ROWS, COLS)


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("definition", [G.DequantDefinition.Affine, G.DequantDefinition.Native])
def test_dense_full_size_bit_exact(cuda, ty, definition):
    vals, _ = ty.block_and_bytes()
    print(f"[case] dense {ty.name} {definition.name} {ROWS}x{COLS}", flush=True)
    raw = synthetic_blocks(int(ty), ROWS * COLS // vals, seed=100 + int(ty))
    check_dense(ty, raw, ROWS, COLS, definition)


@pytest.mark.parametrize("ty", TYPES)
def test_ragged_tail_and_big_endian(cuda, ty):
    vals, nbytes = ty.block_and_bytes()
    rows, cols = 3, 5 * 256  # 15 or 120 blocks: not a multiple of the 256-block stage
    raw = synthetic_blocks(int(ty), rows * cols // vals, seed=7)
    check_convert(ty, raw, rows, cols)
    check_convert(ty, raw, rows, cols, G.Endian.Big)
    check_dense(ty, raw, rows, cols, G.DequantDefinition.Native, G.Endian.Big)
    check_dense(ty, raw, rows, cols, G.DequantDefinition.Affine)


def test_unaligned_payload_takes_the_2_byte_path(cuda):
    ty = G.GgmlType.Q4_0
    raw = synthetic_blocks(int(ty), 512, seed=3)
    big = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
    big[2:2 + raw.size] = dev_u8(raw)
    desc = desc_for(ty, 1, 512 * 32)
    a = G.convert_affine(desc, big[2:2 + raw.size])
    w, s, b = orc.gguf_convert_affine(int(ty), raw)
    assert np.array_equal(words_bytes(a.weights).reshape(-1), w)


def test_boundary_blocks(cuda):
    one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    q40 = np.full(18, 0xFF, np.uint8)
    q40[0:2] = one
    a = G.convert_affine(desc_for(G.GgmlType.Q4_0, 1, 32), dev_u8(q40))
    assert (words_bytes(a.weights) == 0xFFFFFFFF).all()
    q80 = np.full(34, 0xFF, np.uint8)
    q80[0:2] = one
    a = G.convert_affine(desc_for(G.GgmlType.Q8_0, 1, 32), dev_u8(q80))
    assert (words_bytes(a.weights) == 0x7F7F7F7F).all()
    for ty in (G.GgmlType.Q8_0, G.GgmlType.Q4K):
        vals, nbytes = ty.block_and_bytes()
        z = np.zeros(nbytes, np.uint8)
        for d in G.DequantDefinition:
            out = G.dequantize(desc_for(ty, 1, vals), dev_u8(z), definition=d, dtype=torch.float32)
            assert (out == 0).all()


def test_q4k_f16_rounding_exhaustive(cuda):
    """Every finite f16 d and dmin against every 6-bit scale/min: f16(d*sc) and
    f16(-dmin*m) must match the oracle bit for bit (the only inexact step of
    the Q4_K affine route)."""
    d = np.arange(0, 0x7C00, dtype=np.uint16)  # positive finite f16 patterns
    d = np.concatenate([d, d | 0x8000])
    nsb = d.size
    rng = np.random.default_rng(0)
    raw = rng.integers(0, 256, size=(nsb, 144), dtype=np.uint8)
    raw[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    raw[:, 2:4] = d[::-1].copy().view(np.uint8).reshape(nsb, 2)
    # cycle the 12 scale bytes so that all 64 values of every 6-bit field occur
    for j in range(12):
        raw[:, 4 + j] = (np.arange(nsb) * (j + 1) * 7 + j) & 0xFF
    raw = raw.reshape(-1)
    check_convert(G.GgmlType.Q4K, raw, nsb, 256)
    check_dense(G.GgmlType.Q4K, raw, nsb, 256, G.DequantDefinition.Affine)
    check_dense(G.GgmlType.Q4K, raw, nsb, 256, G.DequantDefinition.Native)


def test_converted_tensor_feeds_quantized_matmul(cuda):
    """GGUF -> affine (g32, f16) -> qmv equals x @ dense-dequant^T within tolerance."""
    from eredu_amd import quantized_matmul
    from tests.fixtures import dev_bf16, host_f32, synthetic_x

    for ty in TYPES:
        rows, cols = 512, 4096
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), rows * cols // vals, seed=11)
        a = G.convert_affine(desc_for(ty, rows, cols), dev_u8(raw))
        for M in (1, 4, 40):
            xb = synthetic_x(M, cols, M)
            y = quantized_matmul(dev_bf16(xb), a.weights, a.scales, a.biases, transpose=True,
                                 group_size=a.group_size, bits=a.bits)
            dense = orc.gguf_dequant_f32(int(ty), raw, 0).astype(np.float64).reshape(rows, cols)
            ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ dense.T
            ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, True)
            assert ok, (ty, M, worst)


def test_errors(cuda):
    ty = G.GgmlType.Q4_0
    raw = dev_u8(np.zeros(18 * 4, np.uint8))
    with pytest.raises(EreduError, match="payload length"):
        G.convert_affine(G.TensorDescriptor("x", [64, 1], ty, 18 * 4), raw[:36])
    with pytest.raises(EreduError, match="group size"):
        G.convert_affine(G.TensorDescriptor("x", [48, 1], ty, 18 * 4), raw)


# ----------------------------------------------------------- native linear
# y = x . W^T straight from the blocks; reference: the oracle's native dense
# decode (bit-exact with the device's, tested above) multiplied in fp64.
# Tolerance: the matmul rule |y - y_ref| <= 1e-2 RMS(y_ref) + 1/2 ulp_bf16.

def swap_f16_headers(ty, raw):
    """Byte-swap every block's f16 d (and Q4_K's dmin), the fields the endian
    switch applies to."""
    _, nbytes = ty.block_and_bytes()
    b = raw.reshape(-1, nbytes).copy()
    heads = [0, 2] if ty == G.GgmlType.Q4K else [0]
    for h in heads:
        b[:, [h, h + 1]] = b[:, [h + 1, h]]
    return b.reshape(-1)


# (type, K): Q4_K rows of 5, 13 and 16 superblocks (the MFMA kernel's four
# waves per tile take 2/2/1/0, 4/4/4/1 and 4 each, against a four-deep load
# ring) and of 33 (eight waves: 5 each, the last one none, against a two-deep
# ring); Q8_0 rows of 130 and 129 blocks, whose runs are not whole 16-byte
# words (the 2-byte staging path; the Llama shapes below take the 16-byte one).
# N = 390 leaves a partial tile of rows; M = 11 takes two launches (8 + 3).
LINEAR_CASES = [(G.GgmlType.Q4K, 1280), (G.GgmlType.Q4K, 3328), (G.GgmlType.Q4K, 4096), (G.GgmlType.Q4K, 8448),
                (G.GgmlType.Q8_0, 4160), (G.GgmlType.Q8_0, 4128)]


@pytest.mark.parametrize("ty,K", LINEAR_CASES, ids=[f"{t.name}-K{k}" for t, k in LINEAR_CASES])
@pytest.mark.parametrize("M", [1, 2, 5, 8, 11])
@pytest.mark.parametrize("endian", [G.Endian.Little, G.Endian.Big])
def test_native_linear(cuda, ty, K, M, endian):
    N = 390
    print(f"[case] native linear {ty.name} M={M} N={N} K={K} endian={endian.name}", flush=True)
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), N * K // vals, seed=M + int(ty))
    if endian == G.Endian.Big:
        raw = swap_f16_headers(ty, raw)  # same block values, stored big-endian
    desc = desc_for(ty, N, K)
    rng = np.random.default_rng(M)
    xb = orc.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    y = G.linear(x, desc, dev_u8(raw), endian)
    torch.cuda.synchronize()
    W = orc.gguf_dequant_f32(int(ty), raw, int(G.DequantDefinition.Native),
                             big_endian=endian == G.Endian.Big).reshape(N, K).astype(np.float64)
    y_ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ W.T
    got = (host_bits16(y).astype(np.uint32) << 16).view(np.float32)
    ok, worst, _ = orc.matmul_within_tolerance(got, y_ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


@pytest.mark.parametrize("ty", [G.GgmlType.Q4K, G.GgmlType.Q8_0])
def test_native_linear_llama_shapes(cuda, ty):
    """Decode shapes of a Llama-3-8B checkpoint: q (4096 x 4096), down (4096 x 14336; 7 superblocks per wave of
    the Q4_K MFMA kernel's eight, three turns of its two-deep load ring and one more)."""
    vals, _ = ty.block_and_bytes()
    for N, K in [(4096, 4096), (4096, 14336)]:
        raw = synthetic_blocks(int(ty), N * K // vals, seed=N + K)
        xb = orc.f32_to_bf16_bits(np.random.default_rng(K).standard_normal((1, K)).astype(np.float32))
        x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
        y = G.linear(x, desc_for(ty, N, K), dev_u8(raw))
        W = orc.gguf_dequant_f32(int(ty), raw, int(G.DequantDefinition.Native)).reshape(N, K).astype(np.float64)
        y_ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ W.T
        got = (host_bits16(y).astype(np.uint32) << 16).view(np.float32)
        ok, worst, _ = orc.matmul_within_tolerance(got, y_ref, out_is_bf16=True)
        assert ok, f"{N}x{K}: max|err|/RMS = {worst:.3e}"


@pytest.mark.parametrize("M", [1, 3])
def test_native_q4k_linear_long_rows(cuda, M):
    """Q4_K rows of 84480 values: one staged activation row (169 KB) exceeds a
    workgroup's LDS, so the VALU kernel q4k_linear takes the product."""
    ty, N, K = G.GgmlType.Q4K, 20, 256 * 330
    print(f"[case] native linear long rows M={M} N={N} K={K}", flush=True)
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), N * K // vals, seed=K + M)
    xb = orc.f32_to_bf16_bits(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    y = G.linear(x, desc_for(ty, N, K), dev_u8(raw))
    W = orc.gguf_dequant_f32(int(ty), raw, int(G.DequantDefinition.Native)).reshape(N, K).astype(np.float64)
    y_ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ W.T
    got = (host_bits16(y).astype(np.uint32) << 16).view(np.float32)
    ok, worst, _ = orc.matmul_within_tolerance(got, y_ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"
