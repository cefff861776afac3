"""IQ4_NL / IQ4_XS on the device: dense dequant bit-exact against the oracle
(pinned by llama.cpp's vectors in tests/test_oracle_iq4.py) and against those
vectors themselves; the native linear against the fp64 product with the
closed-form decode, within the matmul rule; routing (the blocks stay native,
no affine form)."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_u8, golden_iq_rows, host_f32, synthetic_blocks, synthetic_x
from tests.test_gpu_gguf import check_dense, desc_for
from tests.test_oracle_iq4 import _closed_form

pytestmark = pytest.mark.gpu

T = G.GgmlType
IQ4 = [T.IQ4NL, T.IQ4XS]


def to_big_endian(ty, raw):
    """d (and IQ4_XS's u16 of high scale bits) byte-swapped."""
    _, nbytes = ty.block_and_bytes()
    b = raw.reshape(-1, nbytes).copy()
    for off in ([0] if ty == T.IQ4NL else [0, 2]):
        b[:, [off, off + 1]] = b[:, [off + 1, off]]
    return b.reshape(-1)


@pytest.mark.parametrize("ty", IQ4)
def test_llama_cpp_vectors_on_device(cuda, ty):
    raw, expected = golden_iq_rows()[int(ty)]
    vals, _ = ty.block_and_bytes()
    out = G.dequantize(desc_for(ty, 2, vals), dev_u8(np.frombuffer(raw, np.uint8).copy()), dtype=torch.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(out.cpu().numpy().reshape(-1).astype(np.float16).view(np.uint16), expected)


@pytest.mark.parametrize("ty", IQ4)
def test_dense_full_size_bit_exact(cuda, ty):
    vals, _ = ty.block_and_bytes()
    print(f"[case] dense {ty.name} 4096x14336", flush=True)
    raw = synthetic_blocks(int(ty), 4096 * 14336 // vals, seed=400 + int(ty))
    check_dense(ty, raw, 4096, 14336, G.DequantDefinition.Affine)
    check_dense(ty, raw, 4096, 14336, G.DequantDefinition.Native)


@pytest.mark.parametrize("ty", IQ4)
def test_dense_ragged_big_endian_unaligned(cuda, ty):
    vals, _ = ty.block_and_bytes()
    per_wg = 256 if vals == 32 else 32
    for rows, cols in ((3, 5 * 256), (1, (2 * per_wg + 1) * vals)):
        print(f"[case] dense {ty.name} {rows}x{cols}", flush=True)
        raw = synthetic_blocks(int(ty), rows * cols // vals, seed=rows + cols)
        check_dense(ty, raw, rows, cols, G.DequantDefinition.Native)
        check_dense(ty, raw, rows, cols, G.DequantDefinition.Native, G.Endian.Big)
    raw = synthetic_blocks(int(ty), 3 * per_wg, seed=5)
    buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + raw.size] = dev_u8(raw)
    out = G.dequantize(desc_for(ty, 1, 3 * per_wg * vals), buf[2:2 + raw.size], dtype=torch.float32)
    assert np.array_equal(out.cpu().numpy().reshape(-1).view(np.uint32), orc.gguf_dequant_f32(int(ty), raw).view(np.uint32))


def run_linear(ty, N, K, M, seed, endian=G.Endian.Little, rel=1e-2, w_bf16_rel=None):
    """y = x·Wᵀ against the fp64 product with the closed-form W, within the
    matmul rule at `rel`; with `w_bf16_rel`, also against the product with W
    rounded to bf16 (what the matrix cores take) at that bound."""
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), N * K // vals, seed=seed)
    stored = to_big_endian(ty, raw) if endian == G.Endian.Big else raw
    desc = G.TensorDescriptor("blk.0.ffn_down.weight", [K, N], ty, stored.size)
    xb = synthetic_x(M, K, seed + 1)
    y = host_f32(G.linear(dev_bf16(xb), desc, dev_u8(stored), endian))
    xf = orc.bf16_bits_to_f32(xb).astype(np.float64)
    w = _closed_form(int(ty), raw).reshape(N, K)
    ok, worst, _ = orc.matmul_within_tolerance(y, xf @ w.T, True, rel=rel)
    assert ok, (ty.name, N, K, M, endian, worst)
    if w_bf16_rel is not None:
        wb = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(w.astype(np.float32))).astype(np.float64)
        ok, worst, _ = orc.matmul_within_tolerance(y, xf @ wb.T, True, rel=w_bf16_rel)
        assert ok, (ty.name, "bf16 W", N, K, M, worst)


@pytest.mark.parametrize("ty,K", [(T.IQ4NL, 4096), (T.IQ4NL, 4128), (T.IQ4XS, 1280), (T.IQ4XS, 4096),
                                  (T.IQ4XS, 14336)])
@pytest.mark.parametrize("M", [1, 3, 8, 11])
def test_native_linear(cuda, ty, K, M):
    print(f"[case] native {ty.name} N=390 K={K} M={M}", flush=True)
    run_linear(ty, 390, K, M, seed=K + M)


@pytest.mark.parametrize("ty", IQ4)
def test_native_linear_big_endian_and_llama_shape(cuda, ty):
    print(f"[case] native {ty.name} big-endian, 4096x14336", flush=True)
    run_linear(ty, 200, 2048, 2, seed=7, endian=G.Endian.Big)
    run_linear(ty, 4096, 14336, 1, seed=8)


def test_routing_keeps_iq4_native_and_refuses_affine(cuda):
    for ty in IQ4:
        vals, _ = ty.block_and_bytes()
        raw = synthetic_blocks(int(ty), 64 * 512 // vals, seed=3)
        desc = G.TensorDescriptor("w", [512, 64], ty, raw.size)
        nt = G.convert(desc, dev_u8(raw), G.Endian.Little)
        assert isinstance(nt, G.NativeTensor)
        dense = nt.dequantize_f32().cpu().numpy().reshape(-1)
        assert np.array_equal(dense.view(np.uint32), orc.gguf_dequant_f32(int(ty), raw).view(np.uint32))
        with pytest.raises(EreduError, match="no affine conversion"):
            G.convert_affine(desc, dev_u8(raw))


@pytest.mark.parametrize("ty", IQ4)
@pytest.mark.parametrize("M", [12, 130])
def test_native_linear_prefill(cuda, ty, M):
    """M > 8: levels as bytes with f16 group factors (kq_to_bytes), then the
    8-bit matrix-core kernel.  Tolerance 2e-2 RMS: the matrix cores take the
    weights in bf16 (2^-9 relative, as MLX's kernels store dequantized
    weights in the activation type), and these synthetic blocks' random
    6-bit group scales spread |W| over four decades, which a 1e-2 bound over
    ~50k outputs does not always absorb (a model of exactly that rounding,
    without the device, reaches 1.2e-2 on some seeds).  Against the product
    with W rounded to bf16 the bound is the usual 1e-2 (what is left is the
    f16 rounding of the group factor)."""
    print(f"[case] native prefill {ty.name} M={M}", flush=True)
    run_linear(ty, 384, 2048, M, seed=M + 3, rel=2e-2, w_bf16_rel=1e-2)
