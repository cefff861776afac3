"""f16 activations on the matrix-core kernels: the output dtype follows x
(safemlx/src/ops/quantization.rs:190-226), and a float16 model takes the same
decode (qmv) and prefill (qmm) kernels as a bfloat16 one, multiplying in f16
(codes as the exact f16 images 1024 + q in decode, weights dequantized and
rounded to f16 in prefill).  Parity against the fp64 oracle on the same packed
inputs at the configs[1] decode shapes and configs[2] prefill shapes (64-row
subsets at the prefill sizes), with bf16 and f16 scales.

Tolerance (the north star's rule, written here): elementwise
|y - y_ref| <= 1e-2 * RMS(y_ref) + 1/2 ulp_bf16(y_ref) -- the half-ulp term is
the bf16 one, larger than f16's, so the bound is the bf16 outputs' bound."""
import numpy as np
import pytest
import torch

from eredu_amd import quantized_matmul_batched, quantized_matmul_with_mode
from oracle import oracle as orc
from tests.fixtures import dev_f16, dev_param, dev_words, host_bits16, host_f32, synthetic_linear, synthetic_x
from tests.test_gpu_matmul import run_case

pytestmark = pytest.mark.gpu

LLAMA_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def f16_x(M, K, seed):
    """f16 bit patterns of x ~ N(0, 1) (the bf16 draw of the other tests, widened)."""
    return orc.bf16_bits_to_f32(synthetic_x(M, K, seed)).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("N,K", LLAMA_SHAPES)
@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("bits", [4, 8])
def test_qmv_f16_llama_shapes(cuda, M, N, K, bits):
    run_case(M, N, K, 64, bits, xdt=orc.F16, seed=N + K + M + bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_qmv_f16_contract_grid(cuda, bits, gs, sdt, M):
    run_case(M, 128, 2048, gs, bits, sdt=sdt, xdt=orc.F16, seed=bits * gs + M + 3)


@pytest.mark.parametrize("K,bits,gs", [(96, 4, 32), (4160, 4, 64), (4224, 8, 128), (160, 8, 32)])
@pytest.mark.parametrize("M", [1, 3])
def test_qmv_f16_ragged_k(cuda, K, bits, gs, M):
    run_case(M, 48, K, gs, bits, xdt=orc.F16, seed=K + bits + gs + M)


def test_qmv_f16_activations_too_large_for_lds(cuda):
    # 16 rows x 14336: the activations do not fit one workgroup's LDS, so the
    # register variant (activations from global memory) runs
    run_case(16, 256, 14336, 64, 4, xdt=orc.F16, seed=5)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,K", LLAMA_SHAPES)
def test_qmm_f16_prefill_config2(cuda, N, K, bits):
    """M in {128, 512} (split K and unsplit plans), a 64-row subset checked."""
    w, s, b = synthetic_linear(N, K, 64, bits, seed=N + 5 * K + bits)
    W = orc.affine_dequant_f64(w, s, b, orc.BF16, N, K, 64, bits)
    wd, sd, bd = dev_words(w), dev_param(s, orc.BF16), dev_param(b, orc.BF16)
    for M in (128, 512):
        print(f"[case] f16 prefill M={M} N={N} K={K} bits={bits}", flush=True)
        xh = f16_x(M, K, seed=M + N + bits)
        y = quantized_matmul_with_mode(dev_f16(xh), wd, sd, bd, True, 64, bits)
        torch.cuda.synchronize()
        assert y.dtype == torch.float16 and tuple(y.shape) == (M, N)
        rng = np.random.default_rng(M + K)
        rows = np.unique(np.concatenate([rng.choice(M, 64, replace=False), [0, 127, M - 1]]))
        ref = xh[rows].view(np.float16).astype(np.float64) @ W.T
        ok, worst, _ = orc.matmul_within_tolerance(host_f32(y)[rows], ref, out_is_bf16=True)
        assert ok, f"M={M}: max|err|/RMS = {worst:.3e}"


@pytest.mark.parametrize("bits,gs,sdt", [(4, 64, orc.F16), (8, 32, orc.BF16), (4, 16, orc.BF16), (3, 16, orc.BF16),
                                         (6, 64, orc.F16)])
def test_qmm_f16_grid(cuda, bits, gs, sdt):
    # M = 300 over 512 columns splits K; the odd widths go through the byte re-pack
    run_case(300, 512, 2048, gs, bits, sdt=sdt, xdt=orc.F16, seed=bits + gs)


@pytest.mark.parametrize("M", [1, 3, 8])
def test_f16_batched_equals_separate_calls_bitwise(cuda, M):
    specs = [(512, 1024), (128, 1024), (128, 1024), (1792, 1024), (1024, 3584)]
    rng_seed = 40 + M
    probs, host = [], []
    for i, (N, K) in enumerate(specs):
        w, s, b = synthetic_linear(N, K, 64, 4, seed=rng_seed + i)
        xh = f16_x(M, K, seed=rng_seed + 10 * i)
        probs.append((dev_f16(xh), dev_words(w), dev_param(s, orc.BF16), dev_param(b, orc.BF16)))
        host.append((xh, w, s, b, N, K))
    ys = quantized_matmul_batched(probs, transpose=True, group_size=64, bits=4)
    torch.cuda.synchronize()
    for (x, w, s, b), y, (xh, wh, sh, bh, N, K) in zip(probs, ys, host):
        assert y.dtype == torch.float16
        y1 = quantized_matmul_with_mode(x, w, s, b, True, 64, 4)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16))
        ref = orc.quantized_matmul_f64(xh, orc.F16, wh, sh, bh, orc.BF16, True, 64, 4, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]


@pytest.mark.parametrize("M", [3, 40])
def test_f16_outputs_round_to_nearest_even(cuda, M):
    """Outputs are the f16 rounding of the f32 sums: with 8-bit codes, power of
    two scales and short activations every product and partial sum is exact,
    so the f32 sum is exact and its RNE f16 image is the only correct result
    (M = 3 on the decode kernel, M = 40 on the prefill kernel)."""
    N, K = 128, 256
    rng = np.random.default_rng(7)
    codes = rng.integers(0, 256, (N, K), dtype=np.uint32)
    w = np.zeros((N, K // 4), dtype=np.uint32)
    for i in range(4):
        w |= codes[:, i::4] << (8 * i)
    s = np.full((N, K // 64), np.float16(2.0 ** -7)).view(np.uint16)
    b = np.full((N, K // 64), np.float16(-1.0)).view(np.uint16)
    x = (rng.integers(-64, 64, (M, K)).astype(np.float16) * np.float16(2.0 ** -4)).view(np.uint16)
    y = quantized_matmul_with_mode(dev_f16(x), dev_words(w), dev_param(s, orc.F16), dev_param(b, orc.F16), True, 64, 8)
    torch.cuda.synchronize()
    ref = x.view(np.float16).astype(np.float64) @ (codes * 2.0 ** -7 - 1.0).T
    assert np.array_equal(host_bits16(y), ref.astype(np.float32).astype(np.float16).view(np.uint16))
