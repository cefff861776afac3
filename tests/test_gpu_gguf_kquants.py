"""Bit-exact parity of the HIP convert / dense kernels for Q4_1, Q5_0, Q5_1,
Q2_K, Q3_K, Q5_K and Q6_K with the oracle (itself pinned by the reference's
golden rows and ggml's decoders in tests/test_oracle_kquants.py), through the
C ABI."""
import numpy as np
import pytest
import torch

from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_u8, golden_rows, host_bits16, synthetic_blocks
from tests.test_gpu_gguf import check_convert, check_dense, desc_for, words_bytes

pytestmark = pytest.mark.gpu

T = G.GgmlType
KTYPES = [T.Q4_1, T.Q5_0, T.Q5_1, T.Q2K, T.Q3K, T.Q5K, T.Q6K]
ROWS, COLS = 4096, 14336


@pytest.mark.parametrize("ty", [T.Q4_1, T.Q2K, T.Q3K, T.Q5K, T.Q6K])
def test_golden_rows_on_device(cuda, ty):
    row = golden_rows()[int(ty)]
    raw = np.frombuffer(row["raw"], dtype=np.uint8).copy()
    vals, _ = ty.block_and_bytes()
    a = G.convert_affine(desc_for(ty, 2, vals), dev_u8(raw))
    torch.cuda.synchronize()
    assert words_bytes(a.weights).tobytes() == row["weight"]
    assert host_bits16(a.scales).tobytes() == row["scales"]
    assert host_bits16(a.biases).tobytes() == row["biases"]
    deq = G.dequantize(desc_for(ty, 2, vals), dev_u8(raw), dtype=torch.float32).cpu().numpy().reshape(-1)
    expected = np.frombuffer(row["dequantized"], dtype=np.uint16).view(np.float16).astype(np.float32)
    got = deq.astype(np.float16).astype(np.float32)
    # eredu-gguf/tests/oracle.rs:103-113 tolerance; exact except for Q6_K, whose
    # fixture column was rounded twice by MLX's f16 kernel
    assert (np.abs(got - expected) <= np.maximum(4.0, np.abs(expected) * 0.002)).all()
    if ty != T.Q6K:
        assert np.array_equal(got, expected)


@pytest.mark.parametrize("ty", [T.Q5_0, T.Q5_1])
def test_q5_golden_rows_on_device(cuda, ty):
    row = golden_rows()[int(ty)]
    raw = np.frombuffer(row["raw"], dtype=np.uint8).copy()
    expected = np.frombuffer(row["weight"], dtype=np.uint16).view(np.float16).astype(np.float32)
    for definition in G.DequantDefinition:
        out = G.dequantize(desc_for(ty, 2, 32), dev_u8(raw), definition=definition, dtype=torch.float32)
        assert np.array_equal(out.cpu().numpy().reshape(-1).astype(np.float16).astype(np.float32), expected)


@pytest.mark.parametrize("ty", KTYPES)
def test_convert_full_size_bit_exact(cuda, ty):
    vals, _ = ty.block_and_bytes()
    print(f"[case] convert {ty.name} {ROWS}x{COLS}", flush=True)
    raw = synthetic_blocks(int(ty), ROWS * COLS // vals, seed=200 + int(ty))
    check_convert(ty, raw, ROWS, COLS)


@pytest.mark.parametrize("ty", KTYPES)
def test_dense_full_size_bit_exact(cuda, ty):
    vals, _ = ty.block_and_bytes()
    print(f"[case] dense {ty.name} {ROWS}x{COLS}", flush=True)
    raw = synthetic_blocks(int(ty), ROWS * COLS // vals, seed=300 + int(ty))
    check_dense(ty, raw, ROWS, COLS, G.DequantDefinition.Affine)
    if ty == T.Q5_1:  # the only one of these with its own native decoder
        check_dense(ty, raw, ROWS, COLS, G.DequantDefinition.Native)


@pytest.mark.parametrize("ty", KTYPES)
def test_ragged_tails_and_big_endian(cuda, ty):
    vals, _ = ty.block_and_bytes()
    per_wg = 256 if vals == 32 else 32  # blocks one workgroup stages
    # fewer blocks than one workgroup; then two full workgroups and one block more
    for rows, cols in ((3, 5 * 256), (1, (2 * per_wg + 1) * vals)):
        print(f"[case] ragged {ty.name} {rows}x{cols}", flush=True)
        raw = synthetic_blocks(int(ty), rows * cols // vals, seed=rows + cols)
        check_convert(ty, raw, rows, cols)
        check_convert(ty, raw, rows, cols, G.Endian.Big)
        check_dense(ty, raw, rows, cols, G.DequantDefinition.Affine)
        check_dense(ty, raw, rows, cols, G.DequantDefinition.Native, G.Endian.Big)


@pytest.mark.parametrize("ty", KTYPES)
def test_unaligned_payload_takes_the_2_byte_path(cuda, ty):
    vals, nbytes = ty.block_and_bytes()
    nblocks = 3 * (256 if vals == 32 else 32)
    raw = synthetic_blocks(int(ty), nblocks, seed=9)
    buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + raw.size] = dev_u8(raw)
    desc = desc_for(ty, 1, nblocks * vals)
    a = G.convert_affine(desc, buf[2:2 + raw.size])
    w, s, b = orc.gguf_convert_affine(int(ty), raw)
    assert np.array_equal(words_bytes(a.weights).reshape(-1), w)
    assert np.array_equal(host_bits16(a.scales).reshape(-1), s)
    assert np.array_equal(host_bits16(a.biases).reshape(-1), b)
    out = G.dequantize(desc, buf[2:2 + raw.size], dtype=torch.float32).cpu().numpy().reshape(-1)
    assert np.array_equal(out.view(np.uint32), orc.gguf_dequant_f32(int(ty), raw).view(np.uint32))


@pytest.mark.parametrize("ty,fields", [(T.Q2K, (80, 82)), (T.Q3K, (108,)), (T.Q5K, (0, 2)), (T.Q6K, (208,))])
def test_f16_rounding_of_scales_exhaustive(cuda, ty, fields):
    """Every finite f16 d (and dmin, reversed) against cycling scale bytes:
    the f16 rounding of d * sc and of the bias (signed for Q3_K / Q6_K) must
    match the oracle bit for bit."""
    d = np.arange(0, 0x7C00, dtype=np.uint16)
    d = np.concatenate([d, d | 0x8000])
    n = d.size
    _, nbytes = ty.block_and_bytes()
    raw = np.random.default_rng(1).integers(0, 256, size=(n, nbytes), dtype=np.uint8)
    for k, off in enumerate(fields):
        raw[:, off:off + 2] = (d if k == 0 else d[::-1].copy()).view(np.uint8).reshape(n, 2)
    scale_bytes = {T.Q2K: range(0, 16), T.Q3K: range(96, 108), T.Q5K: range(4, 16), T.Q6K: range(192, 208)}[ty]
    for j, col in enumerate(scale_bytes):
        raw[:, col] = (np.arange(n) * (j + 1) * 7 + j) & 0xFF
    raw = raw.reshape(-1)
    check_convert(ty, raw, n, 256)
    check_dense(ty, raw, n, 256, G.DequantDefinition.Affine)


def test_converted_kquants_feed_quantized_matmul(cuda):
    """GGUF -> affine (2/3/5/6-bit, groups 16/32, f16) -> quantized_matmul
    equals x @ dense-dequant^T within the matmul rule."""
    from eredu_amd import quantized_matmul
    from tests.fixtures import dev_bf16, host_f32, synthetic_x

    for ty in KTYPES:
        rows, cols = 384, 2048
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), rows * cols // vals, seed=12)
        a = G.convert_affine(desc_for(ty, rows, cols), dev_u8(raw))
        dense = orc.gguf_dequant_f32(int(ty), raw, 0).astype(np.float64).reshape(rows, cols)
        for M in (1, 4, 40):
            print(f"[case] matmul {ty.name} M={M}", flush=True)
            xb = synthetic_x(M, cols, M)
            y = quantized_matmul(dev_bf16(xb), a.weights, a.scales, a.biases, transpose=True,
                                 group_size=a.group_size, bits=a.bits)
            ref = orc.bf16_bits_to_f32(xb).astype(np.float64) @ dense.T
            ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, True)
            assert ok, (ty, M, worst)


def test_convert_routes_the_new_types(cuda):
    """convert.rs:125-140: Q4_1 / Q5_0 / Q2_K / Q3_K are affine in either byte
    order; Q5_1 / Q5_K / Q6_K are affine in big-endian files."""
    for ty, endian in ((T.Q4_1, G.Endian.Little), (T.Q5_0, G.Endian.Little), (T.Q2K, G.Endian.Little),
                       (T.Q3K, G.Endian.Big), (T.Q5_1, G.Endian.Big), (T.Q5K, G.Endian.Big),
                       (T.Q6K, G.Endian.Big)):
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), 4 * 512 // vals, seed=3)
        out = G.convert(desc_for(ty, 4, 512), dev_u8(raw), endian)
        assert isinstance(out, G.AffineTensor), ty
        assert (out.bits, out.group_size) == G.affine_config(ty)
        w, _, _ = orc.gguf_convert_affine(int(ty), raw, big_endian=endian == G.Endian.Big)
        assert np.array_equal(words_bytes(out.weights).reshape(-1), w)
