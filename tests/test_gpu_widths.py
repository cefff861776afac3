"""Parity of the general kernels at the contract's other code widths and group
sizes: bits 3, 5 and 6 (an LSB-first bit stream whose codes straddle words,
eredu-gguf/src/convert.rs:413-427) and 2, and group sizes 16 and 256, which the
fast 4/8-bit kernels at group 32/64/128 do not take (eredu-checkpoint/src/lib.rs:103-122).

Tolerance as in test_gpu_matmul: |y - y_ref| <= 1e-2 * RMS(y_ref) + 1/2 ulp_bf16(y_ref)
against the fp64 product of the same packed inputs; dequantize and quantize are
bit-exact against the oracle.
"""
import numpy as np
import pytest
import torch

from eredu_amd import dequantize_with_mode, gather_qmm_with_mode, quantize_with_mode, quantized_matmul_with_mode
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_param, dev_words, host_bits16, host_f32, synthetic_linear, synthetic_x

pytestmark = pytest.mark.gpu

DT = {orc.BF16: torch.bfloat16, orc.F16: torch.float16, orc.F32: torch.float32}
WIDTHS = [(3, 16), (3, 32), (5, 16), (5, 64), (6, 16), (6, 128), (2, 16), (4, 16), (8, 16), (4, 256), (3, 256)]


@pytest.mark.parametrize("bits,gs", WIDTHS)
@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("M", [1, 5])
def test_matmul_widths(cuda, bits, gs, transpose, M):
    print(f"[case] widths matmul bits={bits} gs={gs} transpose={transpose} M={M}", flush=True)
    N, K = (48, 512) if transpose else (512, 48)
    rows, cols = (N, K) if transpose else (K, N)
    w, s, b = synthetic_linear(rows, cols, gs, bits, seed=bits * 31 + gs + M, scale_dtype=orc.BF16)
    xb = synthetic_x(M, K, seed=bits + gs)
    y = quantized_matmul_with_mode(dev_bf16(xb), dev_words(w), dev_param(s, orc.BF16), dev_param(b, orc.BF16),
                                   transpose, gs, bits)
    torch.cuda.synchronize()
    ref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, orc.BF16, transpose, gs, bits, N, K)
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=True)
    assert y.shape == (M, N)
    assert ok, worst


# qmv_any (transpose, bf16 x, M <= 16): N = 4100 rows take the persistent
# workgroups (4 rows each, at most 4 per CU) through a second pass; M = 7 and
# 16 take launches of 4 activation rows; K = 14336 holds one activation row per
# launch in LDS; f16 scales without biases on a subset.
@pytest.mark.parametrize("bits,gs,sdt,biases", [(3, 64, orc.BF16, True), (5, 32, orc.F16, False),
                                                (6, 16, orc.BF16, True), (2, 128, orc.F16, True),
                                                (8, 256, orc.BF16, False), (4, 16, orc.BF16, True)])
@pytest.mark.parametrize("M,N,K", [(1, 4100, 2048), (7, 4100, 2048), (16, 520, 2048), (3, 260, 14336)])
def test_any_width_decode_shapes(cuda, bits, gs, sdt, biases, M, N, K):
    print(f"[case] qmv_any bits={bits} gs={gs} M={M} N={N} K={K}", flush=True)
    w, s, b = synthetic_linear(N, K, gs, bits, seed=bits * 13 + gs + M + N, scale_dtype=sdt)
    if not biases:
        b = None
    xb = synthetic_x(M, K, seed=bits + gs + M)
    y = quantized_matmul_with_mode(dev_bf16(xb), dev_words(w), dev_param(s, sdt),
                                   dev_param(b, sdt) if b is not None else None, True, gs, bits)
    torch.cuda.synchronize()
    ref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, sdt, True, gs, bits, N, K)
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=True)
    assert y.shape == (M, N)
    assert ok, worst


@pytest.mark.parametrize("bits,gs", WIDTHS)
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16, orc.F32])
def test_dequantize_widths_bit_exact(cuda, bits, gs, sdt):
    print(f"[case] widths dequantize bits={bits} gs={gs} sdt={sdt}", flush=True)
    rows, cols = 40, 768
    w, s, b = synthetic_linear(rows, cols, gs, bits, seed=bits * 7 + gs, scale_dtype=sdt)
    ref = orc.affine_dequant_f32(w, s, b, sdt, rows, cols, gs, bits)
    out = dequantize_with_mode(dev_words(w), dev_param(s, sdt), dev_param(b, sdt), gs, bits, dtype=torch.float32)
    assert np.array_equal(out.cpu().numpy(), ref)
    out16 = dequantize_with_mode(dev_words(w), dev_param(s, sdt), dev_param(b, sdt), gs, bits, dtype=torch.bfloat16)
    assert np.array_equal(host_bits16(out16), orc.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("bits,gs", WIDTHS)
@pytest.mark.parametrize("dtype", [orc.BF16, orc.F32])
def test_quantize_widths_bit_exact(cuda, bits, gs, dtype):
    print(f"[case] widths quantize bits={bits} gs={gs} dtype={dtype}", flush=True)
    rng = np.random.default_rng(bits * 1000 + gs + dtype)
    rows, cols = 37, 768
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[2, :gs] = 0.0  # a constant group
    wt = torch.from_numpy(w).to(DT[dtype]).cuda()
    w_in = wt.float().cpu().numpy()
    wq, s, b = quantize_with_mode(wt, gs, bits)
    torch.cuda.synchronize()
    rq, rs, rb = orc.quantize_affine(w_in, gs, bits, dtype)
    assert np.array_equal(wq.cpu().numpy().view(np.uint32), rq)
    if dtype == orc.F32:
        assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(b.cpu().numpy(), rb)
    else:
        assert np.array_equal(host_bits16(s), rs) and np.array_equal(host_bits16(b), rb)


@pytest.mark.parametrize("bits,gs", [(3, 32), (5, 16), (6, 64)])
@pytest.mark.parametrize("transpose", [True, False])
def test_gather_widths(cuda, bits, gs, transpose):
    print(f"[case] widths gather bits={bits} gs={gs} transpose={transpose}", flush=True)
    E, B, M = 3, 5, 1
    N, K = (64, 256) if transpose else (256, 64)
    rows, cols = (N, K) if transpose else (K, N)
    packs = [synthetic_linear(rows, cols, gs, bits, seed=e + bits, scale_dtype=orc.BF16) for e in range(E)]
    w = torch.stack([dev_words(p[0]) for p in packs])
    s = torch.stack([dev_param(p[1], orc.BF16) for p in packs])
    b = torch.stack([dev_param(p[2], orc.BF16) for p in packs])
    xs = [synthetic_x(M, K, seed=100 + i) for i in range(B)]
    x = torch.stack([dev_bf16(xi) for xi in xs])
    rhs = torch.tensor([2, 0, 1, 2, 0], dtype=torch.int32, device="cuda")
    lhs = torch.tensor([4, 3, 2, 1, 0], dtype=torch.int32, device="cuda")
    y = gather_qmm_with_mode(x, w, s, b, lhs, rhs, transpose, gs, bits, False)
    torch.cuda.synchronize()
    for i in range(B):
        e, xi = int(rhs[i]), xs[int(lhs[i])]
        ref = orc.quantized_matmul_f64(xi, orc.BF16, *packs[e], orc.BF16, transpose, gs, bits, N, K)
        ok, worst, _ = orc.matmul_within_tolerance(host_f32(y[i]), ref, out_is_bf16=True)
        assert ok, (i, worst)


# Prefill (M > 16, transpose, bf16 x) on the matrix cores at the other widths:
# 2/3/5/6-bit codes re-packed to bytes in the workspace and run by the 8-bit
# kernel, and group size 16 in that kernel (two groups per lane's 32 codes) --
# also for 4- and 8-bit codes directly.  N = 384 leaves a partial 256-column
# tile; M = 17 and 130 partial 128-row tiles; 4096 x 4096 at M = 128 splits K.
PREFILL = [(2, 16, orc.BF16, True), (3, 16, orc.F16, True), (3, 64, orc.BF16, False), (5, 32, orc.F16, True),
           (5, 128, orc.BF16, True), (6, 16, orc.BF16, True), (6, 32, orc.F16, False), (4, 16, orc.BF16, True),
           (8, 16, orc.F16, True)]


@pytest.mark.parametrize("bits,gs,sdt,biases", PREFILL)
@pytest.mark.parametrize("M,N,K", [(17, 384, 1024), (130, 256, 2048), (128, 4096, 4096)])
def test_prefill_widths_on_matrix_cores(cuda, bits, gs, sdt, biases, M, N, K):
    print(f"[case] prefill widths bits={bits} gs={gs} M={M} N={N} K={K}", flush=True)
    w, s, b = synthetic_linear(N, K, gs, bits, seed=bits * 17 + gs + M + N, scale_dtype=sdt)
    if not biases:
        b = None
    xb = synthetic_x(M, K, seed=bits + gs + M + 1)
    y = quantized_matmul_with_mode(dev_bf16(xb), dev_words(w), dev_param(s, sdt),
                                   dev_param(b, sdt) if b is not None else None, True, gs, bits)
    torch.cuda.synchronize()
    rows = np.arange(N) if N <= 512 else np.random.default_rng(M).choice(N, 96, replace=False)
    ref = orc.quantized_matmul_f64(xb, orc.BF16, w[rows], s[rows], None if b is None else b[rows], sdt, True, gs,
                                   bits, len(rows), K)
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y)[:, rows], ref, out_is_bf16=True)
    assert y.shape == (M, N)
    assert ok, worst


def test_prefill_odd_width_in_weight_slices(cuda):
    """More weight rows than one 64 MiB slice of byte codes (16384 rows at
    K = 4096): two slices, each writing its columns of y (split K, the
    reduce writing at y's row stride)."""
    from tests.fixtures import device_random_linear, host_rows

    print("[case] prefill 6-bit g16 N=16640 K=4096 M=24", flush=True)
    N, K, M, bits, gs = 16640, 4096, 24, 6, 16
    w, s, b = device_random_linear(N, K, gs, bits, seed=5)
    xb = synthetic_x(M, K, seed=6)
    y = quantized_matmul_with_mode(dev_bf16(xb), w, s, b, True, gs, bits)
    torch.cuda.synchronize()
    rows = np.concatenate([np.arange(0, 32), np.arange(16352, 16416), np.arange(N - 32, N)])
    wr, sr, br = host_rows(w, s, b, rows)
    ref = orc.quantized_matmul_f64(xb, orc.BF16, wr, sr, br, orc.BF16, True, gs, bits, len(rows), K)
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y)[:, rows], ref, out_is_bf16=True)
    assert ok, worst
